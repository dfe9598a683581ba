"""GPU parity of the dense Marlin op (``marlin.mul`` / ``marlin_hip_mul``, reference
marlin/__init__.py:61-75, 134-226) against the CPU oracle: the reference's tile
rules, ragged batches, both scale modes, the Llama-2-7B decode shapes on column
slices, split-K determinism, graph replay, the ``Layer`` module and the reference
benchmark's call site (kernel_bench/bench.py:46-55, 175-188)."""
import numpy as np
import pytest
import torch

from csed499ii_amd import marlin, synth
from oracle import sm24_oracle as o
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _dense_weight(K, N, g, seed):
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    _, s, _ = synth.quantize(w, g)
    B, sp = marlin.pack_dense(w.to(DEV), s.to(DEV), g)
    return {"B": B, "s": sp, "K": K, "N": N, "g": g}


def _run(A, wt, thread_k=-1, thread_n=-1):
    C = torch.full((A.shape[0], wt["N"]), float("nan"), dtype=torch.half, device=DEV)
    ws = torch.zeros(max(wt["N"] // 128 * 16, 16), dtype=torch.int32, device=DEV)
    marlin.mul(A, wt["B"], C, wt["s"], ws, thread_k, thread_n)
    torch.cuda.synchronize()
    return C


def _oracle(A, wt, c0=0, nc=None):
    """Oracle product on chunks [c0, c0 + nc) (64 columns each; the dense layout and
    both scale permutations are self-contained per 64 columns)."""
    K, N, g = wt["K"], wt["N"], wt["g"]
    nc = N // 64 if nc is None else nc
    B = wt["B"].cpu().numpy().reshape(K // 16, 2 * N)[:, 128 * c0:128 * (c0 + nc)]
    s = wt["s"].cpu().numpy()[:, 64 * c0:64 * (c0 + nc)]
    W = o.dense_dequant(np.ascontiguousarray(B), np.ascontiguousarray(s), K, 64 * nc, g)
    return o.gemm(A.cpu().numpy(), W)


@pytest.mark.parametrize("M,N,K,g", [(1, 256, 128, -1), (16, 512, 1024, 128), (5, 256, 256, 128),
                                     (17, 512, 512, -1), (32, 256, 1024, 128), (33, 512, 384, 128),
                                     (64, 768, 256, -1), (130, 512, 1024, 128), (300, 256, 2048, -1)])
def test_dense_against_oracle(M, N, K, g):
    wt = _dense_weight(K, N, g, M + N + K)
    A = synth.make_activation(M, K, M + 7, device=DEV)
    C = _run(A, wt)
    assert_close(C.cpu().numpy(), _oracle(A, wt), f"dense M={M} N={N} K={K} g={g}")
    assert torch.equal(_run(A, wt), C), "repeated dense calls differ"


@pytest.mark.parametrize("M,tile", [(1, (128, 128)), (16, (128, 128)), (16, (64, 256)), (48, (64, 256))])
def test_dense_reference_tiles(M, tile):
    wt = _dense_weight(1024, 512, -1, 40 + M)
    A = synth.make_activation(M, 1024, 41 + M, device=DEV)
    assert_close(_run(A, wt, *tile).cpu().numpy(), _oracle(A, wt), f"dense tiles M={M} {tile}")


def test_dense_shape_errors_raise():
    wt = _dense_weight(1024, 512, -1, 5)
    A = synth.make_activation(32, 1024, 5, device=DEV)
    with pytest.raises(RuntimeError, match="No kernel implementation for thread_k=128, thread_n=128"):
        _run(A, wt, 128, 128)
    with pytest.raises(RuntimeError, match=r"Problem \(m=32, n=512, k=1024\) not compatible"):
        _run(A, wt, 64, 384)


@pytest.mark.parametrize("K,N", [(4096, 12288), (4096, 4096), (4096, 22016), (11008, 4096)])
@pytest.mark.parametrize("M", [1, 16])
def test_dense_llama7b_slices(K, N, M):
    """The Llama-2-7B decode shapes (the reference benchmark's dense column) on the
    first, middle and last column slices; repeated calls bit-identical."""
    wt = _dense_weight(K, N, 128, K + N)
    A = synth.make_activation(M, K, 90 + M, device=DEV)
    C = _run(A, wt)
    assert torch.isfinite(C).all()
    assert torch.equal(_run(A, wt), C)
    chunks = N // 64
    for c0 in (0, chunks // 2 - 1, chunks - 2):
        assert_close(C[:, 64 * c0:64 * (c0 + 2)].cpu().numpy(), _oracle(A, wt, c0, 2), f"dense {K}x{N} M={M}")


def test_dense_graph_replay_matches_eager():
    wt = _dense_weight(4096, 4096, 128, 77)
    A = synth.make_activation(8, 4096, 78, device=DEV)
    ws = torch.zeros(4096 // 128 * 16, dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C_eager = torch.empty(8, 4096, dtype=torch.half, device=DEV)
        marlin.mul(A, wt["B"], C_eager, wt["s"], ws)  # sizes the stream's split-K scratch
    torch.cuda.synchronize()
    C = torch.zeros(8, 4096, dtype=torch.half, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(3):
            marlin.mul(A, wt["B"], C, wt["s"], ws)
    for _ in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_eager)


def test_dense_layer_forward():
    K, N = 1024, 512
    gen = torch.Generator().manual_seed(3)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    _, s, ref = synth.quantize(w, 128)
    layer = marlin.Layer(K, N, groupsize=128).to(DEV)
    lin = torch.nn.Linear(K, N)
    lin.weight.data = ref.to(DEV)
    layer.pack(lin, s.to(DEV))
    x = torch.randn((2, 3, K), generator=gen).half().to(DEV)
    y = layer(x)
    assert y.shape == (2, 3, N)
    wt = {"B": layer.B, "s": layer.s, "K": K, "N": N, "g": 128}
    assert_close(y.reshape(6, N).cpu().numpy(), _oracle(x.reshape(6, K), wt), "dense Layer.forward")


@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (16, 4096, 12288)])
def test_dense_reference_bench_call_site(m, k, n):
    """get_marlin_prob / benchmark_dense_marlin (kernel_bench/bench.py:46-55, 175-188):
    a 1-D int32 B of K*N/8 random words, zero scales [K/128, N], workspace
    C.shape[1] // 128 * 16, positional -1, -1, sms: C == 0; then random scales in the
    same buffer give the oracle's product of the same random codes."""
    sms = torch.cuda.get_device_properties(torch.device(DEV)).multi_processor_count
    gen = torch.Generator(device=DEV).manual_seed(k + n)
    A = torch.randn((m, k), dtype=torch.half, device=DEV, generator=gen)
    B = torch.randint(-(2 ** 31), 2 ** 31, (k * n // 8,), dtype=torch.int32, device=DEV, generator=gen)
    C = torch.zeros((m, n), dtype=torch.half, device=DEV)
    s = torch.zeros((k // 128, n), dtype=torch.half, device=DEV)
    workspace = torch.zeros(C.shape[1] // 128 * 16, device=torch.device(DEV), dtype=torch.int32)
    marlin.mul(A, B, C, s, workspace, -1, -1, sms)
    torch.cuda.synchronize()
    assert torch.equal(C, torch.zeros_like(C))
    s.copy_((torch.rand(s.shape, device=DEV, generator=gen) * 0.01 + 1e-3).half())
    marlin.mul(A, B, C, s, workspace, -1, -1, sms)
    torch.cuda.synchronize()
    wt = {"B": B, "s": s, "K": k, "N": n, "g": 128}
    chunks = n // 64
    for c0 in (0, chunks - 2):
        assert_close(C[:, 64 * c0:64 * (c0 + 2)].cpu().numpy(), _oracle(A, wt, c0, 2), f"dense bench {m}x{k}x{n}")


# ---- large batches: the MFMA-bound dense kernel (marlin_dense_prefill_kernel) ----

@pytest.mark.parametrize("M,N,K,g", [(65, 512, 128, 128), (128, 512, 1024, -1), (300, 1024, 2048, 128),
                                     (257, 1536, 384, -1), (512, 4096, 4096, 128), (1000, 2048, 640, 128),
                                     (129, 512, 8192, 128), (700, 512, 4096, -1)])
def test_dense_large_m_against_oracle(M, N, K, g):
    """Ragged row tiles, 1 to 64 k-steps, per-column and grouped scales, several
    column tiles, and few tiles with long K (split K through the stream's scratch);
    repeated calls bit-identical (split-K partials added in split order)."""
    wt = _dense_weight(K, N, g, 3 * M + N + K)
    A = synth.make_activation(M, K, M + 11, device=DEV)
    C = _run(A, wt)
    chunks = N // 64
    for c0 in sorted({0, chunks // 2 - 1, chunks - 2}):
        assert_close(C[:, 64 * c0:64 * (c0 + 2)].cpu().numpy(), _oracle(A, wt, c0, 2),
                     f"dense large M={M} N={N} K={K} g={g} chunk {c0}")
    assert torch.equal(_run(A, wt), C), "repeated dense large-M calls differ"


@pytest.mark.parametrize("M", [512, 2048])
@pytest.mark.parametrize("K,N", [(8192, 10240), (8192, 57344), (28672, 8192)])
def test_dense_large_m_llama70b_slices(K, N, M):
    """Llama-2-70B prefill shapes on dense weights: first, middle and last column
    slices against the oracle (all rows, so the last row tile too)."""
    wt = _dense_weight(K, N, 128, K + N + 1)
    A = synth.make_activation(M, K, 70 + M, device=DEV)
    C = _run(A, wt)
    assert torch.isfinite(C).all()
    chunks = N // 64
    for c0 in (0, chunks // 2 - 1, chunks - 2):
        assert_close(C[:, 64 * c0:64 * (c0 + 2)].cpu().numpy(), _oracle(A, wt, c0, 2), f"dense {K}x{N} M={M}")


def test_dense_large_m_matches_small_batch_path():
    """The same rows through the large-M kernel (M = 96) and through the decode-sized
    kernel (three calls of 32 rows) agree within the GEMM tolerance."""
    wt = _dense_weight(4096, 4096, 128, 5)
    A = synth.make_activation(96, 4096, 6, device=DEV)
    C = _run(A, wt)
    parts = torch.cat([_run(A[32 * i:32 * (i + 1)].contiguous(), wt) for i in range(3)])
    assert_close(C.cpu().numpy(), parts.cpu().numpy(), "dense large-M vs decode-sized")


def test_dense_large_m_graph_replay_split_k():
    """A captured large-M call that splits K (one column tile, K = 8192) replays the
    eager result, with the eager call run first on the capture stream."""
    wt = _dense_weight(8192, 512, 128, 9)
    A = synth.make_activation(128, 8192, 10, device=DEV)
    ws = torch.zeros(512 // 128 * 16, dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C_eager = torch.empty(128, 512, dtype=torch.half, device=DEV)
        marlin.mul(A, wt["B"], C_eager, wt["s"], ws)
    torch.cuda.synchronize()
    C = torch.zeros(128, 512, dtype=torch.half, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(2):
            marlin.mul(A, wt["B"], C, wt["s"], ws)
    for _ in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_eager)
