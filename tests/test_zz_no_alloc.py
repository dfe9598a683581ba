"""marlin_hip_mul_2_4_noalloc, called through the C ABI, against marlin_hip_mul_2_4 (the
entry point it is a variant of) and the CPU oracle: two calls in a row, the second on
a smaller problem, then capture on a stream that has never run a call.  Where both
entry points take the same plan the outputs are bit-identical; where mul_2_4 splits K
(and the no-allocation path does not) they agree within the GEMM tolerance."""
import ctypes

import pytest
import torch

from csed499ii_amd import _lib, marlin, synth
from tests.gpu_util import assert_close, check_slices, to_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _noalloc(A, wt, C, stream=None):
    """One call of marlin_hip_mul_2_4_noalloc through ctypes (prob_m = N, prob_n = M)."""
    M, K = A.shape
    N = wt["N"]
    g = -1 if wt["s"].shape[0] == 1 else K // 2 // wt["s"].shape[0]
    st = (stream or torch.cuda.current_stream()).cuda_stream
    err = _lib.load().marlin_hip_mul_2_4_noalloc(
        ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(wt["B"].data_ptr()), ctypes.c_void_p(wt["meta"].data_ptr()),
        ctypes.c_void_p(C.data_ptr()), ctypes.c_void_p(wt["s"].data_ptr()), N, M, K, g, A.get_device(),
        ctypes.c_void_p(st), -1, -1, -1)
    assert err == _lib.OK, _lib.last_error()


def _mul(A, wt):
    C = torch.full((A.shape[0], wt["N"]), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], torch.zeros(wt["N"] // 128 * 16, dtype=torch.int32,
                                                                      device=DEV))
    return C


# (M, K, N, group): mul_2_4 splits K on the first (decode, 64-column tiles in two
# splits) and the third (large-M kernel, 32 tiles of 64 rows on 256 CUs, split three
# ways); not on the second.
CASES = [(16, 4096, 22016, 128), (4, 4096, 4096, 128), (256, 4096, 4096, -1), (1, 1024, 512, 128)]


def test_noalloc_matches_mul_2_4_two_calls():
    """Two calls in a row, the second smaller: each against mul_2_4 and the oracle."""
    for (M1, K1, N1, g1), (M2, K2, N2, g2) in ((CASES[0], CASES[1]), (CASES[2], CASES[3])):
        for M, K, N, g in ((M1, K1, N1, g1), (M2, K2, N2, g2)):
            wt = synth.make_weight(K, N, 300 + M + K + N, g, device=DEV)
            A = synth.make_activation(M, K, 301 + M, device=DEV)
            C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
            _noalloc(A, wt, C)
            ref = _mul(A, wt)
            torch.cuda.synchronize()
            assert torch.isfinite(C).all()
            assert_close(C.cpu().numpy(), ref.cpu().numpy(), f"noalloc vs mul_2_4 M={M} K={K} N={N}")
            if (M, K, N) in ((4, 4096, 4096), (1, 1024, 512)):  # same plan: same bits
                assert torch.equal(C, ref)
            chunks = N // 64
            check_slices(C, A.cpu().numpy(), to_cpu(wt), (0, chunks // 2 - 2, chunks - 4), 4,
                         f"noalloc M={M} K={K} N={N}")


def test_noalloc_captured_on_fresh_stream():
    """Captured on a stream that has never run a call (so nothing could be allocated
    for it): replays equal the eager no-allocation result bit for bit, with eager work
    and synchronisations between the replays."""
    wt = synth.make_weight(4096, 12288, 321, 128, device=DEV)
    A = synth.make_activation(8, 4096, 322, device=DEV)
    C_eager = torch.empty(8, 12288, dtype=torch.half, device=DEV)
    _noalloc(A, wt, C_eager)
    torch.cuda.synchronize()
    C = torch.zeros_like(C_eager)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _noalloc(A, wt, C, stream=s)
    for _ in range(3):
        C.fill_(float("nan"))
        other = _mul(A, wt)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_eager)
        assert_close(C.cpu().numpy(), other.cpu().numpy(), "captured noalloc vs mul_2_4")


def test_capture_on_fresh_stream_runs_unsplit():
    """A split-K call captured on a stream that has never run a call cannot allocate
    that stream's scratch: it is captured without a K split.  Replays match the
    unsplit (no-allocation) product bit for bit and the oracle within tolerance."""
    assert marlin.plan_2_4(16, 4096, 22016)["splits"] > 1  # the eager plan splits K (tail tiles)
    wt = synth.make_weight(4096, 22016, 511, 128, device=DEV)
    A = synth.make_activation(16, 4096, 512, device=DEV)
    C_unsplit = torch.empty(16, 22016, dtype=torch.half, device=DEV)
    marlin.mul_2_4_noalloc(A, wt["B"], wt["meta"], C_unsplit, wt["s"])
    torch.cuda.synchronize()
    C = torch.zeros(16, 22016, dtype=torch.half, device=DEV)
    ws = torch.zeros(22016 // 128 * 16, dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], ws)
    for _ in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_unsplit)
    check_slices(C, A.cpu().numpy(), to_cpu(wt), (0, 170, 340), 4, "captured unsplit gate_up")


_FIRST_CALL_CAPTURED = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
from csed499ii_amd import _lib, synth
lib = _lib.load()
dev = "cuda:0"
wt = synth.make_weight(4096, 4096, 331, 128, device=dev)
A = synth.make_activation(4, 4096, 332, device=dev)
C = torch.full((4, 4096), float("nan"), dtype=torch.half, device=dev)
C_eager = torch.empty_like(C)
torch.cuda.synchronize()

def call(out, stream):
    err = lib.marlin_hip_mul_2_4_noalloc(
        ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(wt["B"].data_ptr()), ctypes.c_void_p(wt["meta"].data_ptr()),
        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(wt["s"].data_ptr()), 4096, 4, 4096, 64, 0,
        ctypes.c_void_p(stream.cuda_stream), -1, -1, -1)
    assert err == 0, _lib.last_error()

s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):  # the process's first call into the library
    call(C, s)
for _ in range(3):
    C.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    call(C_eager, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert torch.equal(C, C_eager), "replay differs from the eager call"
print("FIRST_CALL_CAPTURED_OK", flush=True)
"""


def test_noalloc_first_call_captured_in_fresh_process():
    """A process whose very first library call is marlin_hip_mul_2_4_noalloc under
    stream capture (so the static zero block is looked up while capturing and no
    clearing launch may be recorded into the graph): replays equal an eager call made
    afterwards, bit for bit.  Runs in a child process (started, not exec'd)."""
    import pathlib
    import subprocess
    import sys

    root = str(pathlib.Path(__file__).resolve().parents[1])
    out = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                         timeout=110)
    assert out.returncode == 0 and "FIRST_CALL_CAPTURED_OK" in out.stdout, out.stdout[-2000:] + out.stderr[-2000:]
