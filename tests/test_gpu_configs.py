"""GPU parity at the benchmark configurations that the other files do not reach: the
Llama-2-70B prefill sweep at full size, calls on two streams at
once, capture on a stream that has no split-K scratch yet, and the reference
benchmark's own call sites (kernel_bench/bench.py).  Every check is against the CPU
oracle, on column slices (every packed operand is self-contained per 64 columns)."""
import numpy as np
import pytest
import torch

from csed499ii_amd import marlin, synth
from tests.gpu_util import assert_close, cached_weight, check_slices, oracle_gemm, to_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

LLAMA70B = {"qkv": (8192, 10240), "o": (8192, 8192), "gate_up": (8192, 57344), "down": (28672, 8192)}


def _ws(N):
    return torch.zeros(max(N // 128 * 16, 16), dtype=torch.int32, device=DEV)


def _mul(A, wt, C=None):
    M, N = A.shape[0], wt["N"]
    if C is None:
        C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], _ws(N))
    return C


# (shape, M), grouped by shape so that each 70B weight is built once: every point of
# the bench's prefill sweep (M in {512, 1024, 2048, 4096}) plus o at M = 4000.  The
# planner's choices (256 CUs): qkv at M = 512 and o at M = 1024 run 64-row tiles
# unsplit, o at M = 512 64-row tiles split in two; down splits 128-row tiles four
# ways at M = 512 and two ways at M = 1024; o at M = 4000 has a ragged last 128-row
# tile; gate_up at M = 4096 is the largest grid (3584 workgroups).
PREFILL_CASES = [(name, M) for name in ("qkv", "o", "down", "gate_up")
                 for M in {"qkv": (512, 1024, 2048, 4096), "o": (512, 1024, 2048, 4000, 4096),
                           "down": (512, 1024, 2048, 4096), "gate_up": (512, 1024, 2048, 4096)}[name]]


@pytest.mark.parametrize("name,M", PREFILL_CASES)
def test_prefill_llama70b_full_size(name, M):
    """BASELINE config 3 at full size: first, middle and last 128-column slices, all
    M rows (so the last row tile too), against the oracle; a repeated call is
    bit-identical (split-K partials are added in split order)."""
    K, N = LLAMA70B[name]
    wt, t = cached_weight(K, N, K + N)
    A = synth.make_activation(M, K, 700 + M, device=DEV)
    C = _mul(A, wt)
    torch.cuda.synchronize()
    assert torch.isfinite(C).all()
    assert torch.equal(_mul(A, wt), C), "repeated prefill calls differ"
    chunks = N // 64
    check_slices(C, A.cpu().numpy(), t, (0, chunks // 2 - 1, chunks - 2), 2, f"prefill {name} M={M}")


def test_two_streams_split_k_overlap():
    """Two layers on two same-priority streams, both planned with split-K (gate_up
    4096x22016 at M = 24 splits in two, Llama-2-70B qkv 8192x10240 at M = 4 in four),
    issued back to back with no synchronisation between them: each stream has its
    own scratch, so both results match the oracle and the sequential results."""
    assert marlin.plan_2_4(24, 4096, 22016)["splits"] == 2
    assert marlin.plan_2_4(4, 8192, 10240)["splits"] == 4
    w1 = synth.make_weight(4096, 22016, 501, 128, device=DEV)
    w2 = synth.make_weight(8192, 10240, 502, 128, device=DEV)
    A1 = synth.make_activation(24, 4096, 503, device=DEV)
    A2 = synth.make_activation(4, 8192, 504, device=DEV)
    ref1, ref2 = _mul(A1, w1), _mul(A2, w2)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    C1 = torch.full_like(ref1, float("nan"))
    C2 = torch.full_like(ref2, float("nan"))
    for _ in range(2):  # the first round grows each stream's scratch, the second reuses it
        torch.cuda.synchronize()
        C1.fill_(float("nan"))
        C2.fill_(float("nan"))
        torch.cuda.synchronize()
        for _ in range(8):
            with torch.cuda.stream(s1):
                _mul(A1, w1, C1)
            with torch.cuda.stream(s2):
                _mul(A2, w2, C2)
        torch.cuda.synchronize()
        assert torch.equal(C1, ref1), "gate_up on stream 1 differs from the sequential result"
        assert torch.equal(C2, ref2), "70B o on stream 2 differs from the sequential result"
    t1, t2 = to_cpu(w1), to_cpu(w2)
    check_slices(C1, A1.cpu().numpy(), t1, (0, 170, 340), 4, "stream 1 gate_up M=24")
    check_slices(C2, A2.cpu().numpy(), t2, (0, 78, 156), 4, "stream 2 qkv M=4")


def test_two_graphs_split_k_concurrent_replays():
    """The scratch rule for graphs: a captured split-K call keeps its capture stream's
    scratch.  The two split-K layers above, each captured (three calls) on its own
    capture stream after an eager call there, are replayed back to back on two other
    streams with no synchronisation between the replays, three rounds with eager work
    and a synchronisation between them: the graphs never share counters or partials,
    so every replay equals its eager result bit for bit."""
    w1 = synth.make_weight(4096, 22016, 501, 128, device=DEV)
    w2 = synth.make_weight(8192, 10240, 502, 128, device=DEV)
    A1 = synth.make_activation(24, 4096, 503, device=DEV)
    A2 = synth.make_activation(4, 8192, 504, device=DEV)
    cs1, cs2 = torch.cuda.Stream(), torch.cuda.Stream()
    C1, C2 = torch.empty(24, 22016, dtype=torch.half, device=DEV), torch.empty(4, 10240, dtype=torch.half, device=DEV)
    eager = []
    for cs, A, w, C in ((cs1, A1, w1, C1), (cs2, A2, w2, C2)):
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cs):
            eager.append(_mul(A, w))  # sizes the capture stream's scratch
    torch.cuda.synchronize()
    graphs = []
    for cs, A, w, C in ((cs1, A1, w1, C1), (cs2, A2, w2, C2)):
        ws = _ws(w["N"])  # allocated (and zeroed) before the capture: nothing but the GEMMs is recorded
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            for _ in range(3):
                marlin.mul_2_4(A, w["B"], w["meta"], C, w["s"], ws)
        graphs.append((g, ws))
    rs1, rs2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        C1.fill_(float("nan"))
        C2.fill_(float("nan"))
        torch.cuda.synchronize()
        for _ in range(4):
            with torch.cuda.stream(rs1):
                graphs[0][0].replay()
            with torch.cuda.stream(rs2):
                graphs[1][0].replay()
        torch.cuda.synchronize()
        assert torch.equal(C1, eager[0]), "graph 1 (gate_up M=24) differs from its eager result"
        assert torch.equal(C2, eager[1]), "graph 2 (70B qkv M=4) differs from its eager result"


# ---- the reference benchmark's call sites (kernel_bench/bench.py) ----

def _problem_24(m, n, k, groupsize, seed):
    """gen_2_4 / get_problem_24 (kernel_bench/bench.py:108-124): a 1-D int32 B of
    K*N/16 random words, a 1-D int16 meta of N*K/16 entries all -4370 (0xEEEE: the
    last two positions of every group of 4), zero scales [1, N] or [K/128, N]."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    B = torch.randint(-(2 ** 31), 2 ** 31, (k * n // 8 // 2,), dtype=torch.int32, device=DEV, generator=g)
    meta = torch.ones((n * k // 16,), dtype=torch.int16, device=DEV) * (-4370)
    if groupsize == -1:
        s = torch.zeros((1, n), dtype=torch.half, device=DEV)
    else:
        s = torch.zeros(((k // 2) // (groupsize // 2), n), dtype=torch.half, device=DEV)
    return B, meta, s


@pytest.mark.parametrize("m,k,n", [(1, 4096, 12288), (16, 4096, 4096), (16, 11008, 4096), (512, 8192, 8192)])
def test_reference_bench_call_sites(m, k, n):
    """benchmark_sparse_marlin (kernel_bench/bench.py:159-173) calls
    mul_2_4(A, B, meta, C, s, workspace, -1, -1, sms) with the operands above, a
    workspace of C.shape[1] // 128 * 16 int32 and sms = multi_processor_count.  Zero
    scales give C == 0 exactly; then random scales in the same buffers give the
    oracle's product of the same random codes."""
    sms = torch.cuda.get_device_properties(torch.device(DEV)).multi_processor_count
    B, meta, s = _problem_24(m, n, k, 128, 900 + m + k)
    A = torch.randn((m, k), dtype=torch.half, device=DEV, generator=torch.Generator(device=DEV).manual_seed(m))
    C = torch.full((m, n), float("nan"), dtype=torch.half, device=DEV)
    workspace = torch.zeros(C.shape[1] // 128 * 16, device=torch.device(DEV), dtype=torch.int32)
    marlin.mul_2_4(A, B, meta, C, s, workspace, -1, -1, sms)
    torch.cuda.synchronize()
    assert torch.equal(C, torch.zeros_like(C)), "zero scales must give a zero product"
    s.copy_((torch.rand(s.shape, device=DEV, generator=torch.Generator(device=DEV).manual_seed(k)) * 0.01 + 1e-3)
            .half())
    marlin.mul_2_4(A, B, meta, C, s, workspace, -1, -1, sms)
    torch.cuda.synchronize()
    t = {"B": B.cpu().numpy(), "meta": meta.cpu().numpy(), "s": s.cpu().numpy(), "K": k, "N": n,
         "groupsize": 128, "bits": 4}
    check_slices(C, A.cpu().numpy(), t, (0, n // 128 - 1, n // 64 - 2), 2, f"bench call site {m}x{k}x{n}")
