"""GPU parity of the 2:4 INT4 GEMM (libmarlin_hip.so via the C ABI) against the
CPU oracle, on the reference's own test shapes (test_2_4.py:91-135, run.py:46),
ragged batches, the benchmark shapes (checked through 256-column slices at full K),
determinism, full overwrite of C and hipGraph replay."""
import numpy as np
import pytest
import torch

from csed499ii_amd import marlin, synth
from tests.gpu_util import REL_MAE, assert_close, oracle_gemm, slice_cols, to_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _problem(M, N, K, g, seed, bits=4):
    wt = synth.make_weight(K, N, seed, g, bits=bits, device=DEV)
    A = synth.make_activation(M, K, seed, device=DEV)
    return wt, A


def _run(wt, A, fn=None, thread_k=-1, thread_m=-1, meta=None):
    fn = fn or (marlin.mul_2_4 if wt["bits"] == 4 else marlin.mul_2_4_w3)
    M, N = A.shape[0], wt["N"]
    C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    ws = torch.zeros(max(N // 128 * 16, 16), dtype=torch.int32, device=DEV)
    fn(A, wt["B"], wt["meta"] if meta is None else meta, C, wt["s"], ws, thread_k, thread_m)
    torch.cuda.synchronize()
    return C


def _check(wt, A, C, what):
    t = to_cpu(wt)
    ref = oracle_gemm(A.cpu().numpy(), t)
    return assert_close(C.cpu().numpy(), ref, what)


def test_reference_correctness_cases():
    """test_2_4.py:91-93: (N, batch, K) = (256, 16, 256) g=-1 tile 128x128 and
    (21504, 16, 4096) g=128 tile 64x256 (the latter checked on column slices)."""
    wt, A = _problem(16, 256, 256, -1, 1)
    C = _run(wt, A, thread_k=128, thread_m=128)
    _check(wt, A, C, "256x16x256")
    wt, A = _problem(16, 21504, 4096, 128, 2)
    C = _run(wt, A, thread_k=64, thread_m=256)
    t = to_cpu(wt)
    for c0 in (0, 160, 332):
        ts = slice_cols(t, c0, 4)
        ref = oracle_gemm(A.cpu().numpy(), ts)
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"21504 slice {c0}")
    assert torch.isfinite(C).all()


@pytest.mark.parametrize("batch", [1, 2, 4, 8, 12, 16, 32, 64])
@pytest.mark.parametrize("tile", [(64, 256), (128, 128)])
def test_reference_tiles(batch, tile):
    """test_2_4.py:95-101 (N=512, K=1024, g=-1).  The reference's (thread_k, thread_m)
    pick a CUDA kernel configuration; here they are checked against the reference's
    rules (an unsupported pair raises, test_kernel_shape_errors_raise) and accepted
    pairs give the same product, computed with the planner's own tile choice for
    this GPU (the tile arguments do not select a kernel)."""
    if batch > 16 and tile == (128, 128):
        pytest.skip("the reference has no 128x128 kernel for more than one batch block")
    wt, A = _problem(batch, 512, 1024, -1, 10 + batch)
    C = _run(wt, A, thread_k=tile[0], thread_m=tile[1])
    _check(wt, A, C, f"tiles batch={batch} {tile}")


@pytest.mark.parametrize("K", [768, 832, 896])
def test_reference_k_stages(K):
    """test_2_4.py:103-106."""
    wt, A = _problem(16, 512, K, -1, K)
    _check(wt, A, _run(wt, A, thread_k=64, thread_m=256), f"K={K}")


@pytest.mark.parametrize("K", [64, 128, 192])
def test_reference_very_few_stages(K):
    """test_2_4.py:108-111 (N=768)."""
    wt, A = _problem(16, 768, K, -1, K + 1)
    _check(wt, A, _run(wt, A, thread_k=64, thread_m=256), f"K={K}")


@pytest.mark.parametrize("N,K", [(256, 512), (256, 1024), (256 * 128, 1024)])
@pytest.mark.parametrize("tile", [(128, 128), (64, 256)])
def test_reference_groups(N, K, tile):
    """test_2_4.py:129-135 (batch 16, g=128)."""
    wt, A = _problem(16, N, K, 128, N + K)
    C = _run(wt, A, thread_k=tile[0], thread_m=tile[1])
    if N <= 4096:
        _check(wt, A, C, f"groups {N}x{K}")
    else:
        t = to_cpu(wt)
        for c0 in (0, 255, 508):
            ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
            assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"groups slice {c0}")


@pytest.mark.parametrize("M", [1, 16, 32])
@pytest.mark.parametrize("g", [-1, 128])
def test_run_py_check_cases(M, g):
    """run.py:46 (N=512, K=1024)."""
    wt, A = _problem(M, 512, 1024, g, 100 + M)
    _check(wt, A, _run(wt, A), f"M={M} g={g}")


@pytest.mark.parametrize("M", [3, 7, 17, 33, 50, 100, 129])
def test_ragged_batches(M):
    wt, A = _problem(M, 1024, 2048, 128, 200 + M)
    _check(wt, A, _run(wt, A), f"M={M}")


@pytest.mark.parametrize("M", [1, 2, 4, 5, 6, 7, 8, 16])
def test_config1_and_decode_o_proj(M):
    """Benchmark config 1 (M=16) and the decode sweep at the O-projection shape (5-8
    rows: the 8-row batch, activation rows staged through LDS)."""
    wt, A = _problem(M, 4096, 4096, 128, 20261019 + M)
    _check(wt, A, _run(wt, A), f"4096^2 M={M}")


@pytest.mark.parametrize("K,N", [(4096, 12288), (4096, 22016), (11008, 4096), (4096, 4096)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16, 24, 32, 64, 90])
def test_decode_sweep_full_size_slices(K, N, M):
    """Full-width calls (every decode tile width and padded batch), checked on
    column slices; repeated calls must be bit-identical (a race between the LDS
    stage buffers shows up as run-to-run differences)."""
    wt, A = _problem(M, N, K, 128, K + N + M)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    for _ in range(4):
        assert torch.equal(_run(wt, A), C), "repeated decode calls differ"
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2 - 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"{K}x{N} M={M} slice {c0}")


_W70 = {}


def _weight70(K, N):
    """One Llama-2-70B weight at a time (device and host copies), reused across M."""
    if (K, N) not in _W70:
        _W70.clear()
        wt = synth.make_weight(K, N, K + N, 128, device=DEV)
        _W70[(K, N)] = (wt, to_cpu(wt))
    return _W70[(K, N)]


@pytest.mark.parametrize("M", [1, 2, 4, 7, 8, 12, 16, 32])
@pytest.mark.parametrize("K,N", [(8192, 10240), (8192, 8192), (28672, 8192), (8192, 57344)])
def test_decode_llama70b_full_size_slices(K, N, M):
    """The Llama-2-70B decode shapes (long K: 32- and 64-column tiles, K unsplit or
    split two or four ways, the tail tiles of 8192x10240 split four ways at M <= 4,
    9-16 rows on the 16-row batch; at M = 32 the widest shape, 8192x57344, runs the
    large-M kernel), checked on column slices; repeated calls must be bit-identical."""
    wt, t = _weight70(K, N)
    A = synth.make_activation(M, K, 70 + M, device=DEV)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    for _ in range(2):
        assert torch.equal(_run(wt, A), C), "repeated decode calls differ"
    chunks = N // 64
    for c0 in (0, chunks // 2 - 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"{K}x{N} M={M} slice {c0}")


@pytest.mark.parametrize("M,N,K,g", [(256, 512, 128, 128), (300, 1024, 256, -1), (257, 512, 192, -1),
                                     (257, 512, 384, -1), (320, 1024, 384, 128),
                                     (384, 1536, 512, 128), (640, 2048, 1024, 128),
                                     (80, 16384, 512, 128), (100, 8192, 512, -1), (160, 4096, 512, 128)])
def test_prefill_kernel_shapes(M, N, K, g):
    """The large-M kernel: ragged row tiles, 1-3 k-steps, per-column and grouped
    scales, several column tiles (every XCD ordering branch).  Problems this small
    have few tiles, so the planner gives them 64-row tiles."""
    wt, A = _problem(M, N, K, g, 900 + M + K)
    C = _run(wt, A)
    _check(wt, A, C, f"prefill M={M} N={N} K={K} g={g}")
    assert torch.equal(_run(wt, A), C), "repeated calls differ"


@pytest.mark.parametrize("M,N,K,g", [(300, 512, 8192, -1), (1000, 2048, 8192, 128), (256, 1024, 4096, 128),
                                     (100, 4096, 4096, 128), (130, 4096, 11008, -1)])
def test_prefill_split_k(M, N, K, g):
    """Large-M kernel split along K (few tiles, long K: the planner picks 3-8 splits
    of 64-row tiles):
    partials handed off through the scratch, reduced by the last split in split order,
    so repeated calls agree bit for bit and the counters return to zero."""
    wt, A = _problem(M, N, K, g, 1700 + M + K)
    C = _run(wt, A)
    _check(wt, A, C, f"prefill split-K M={M} N={N} K={K} g={g}")
    for _ in range(3):
        assert torch.equal(_run(wt, A), C), "repeated split-K calls differ"


@pytest.mark.parametrize("M", [512])
def test_prefill_shape_slices(M):
    wt, A = _problem(M, 8192, 8192, 128, 31)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    t = to_cpu(wt)
    for c0 in (0, 64, 124):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"prefill M={M} slice {c0}")


@pytest.mark.parametrize("M,K,N", [(17, 8192, 57344), (33, 4096, 22016), (33, 8192, 10240), (65, 4096, 4096)])
def test_prefill_from_few_rows(M, K, N):
    """The large-M kernel at the smallest batches routed to it (from 17 rows for the
    widest N at long K, from 33 for the widest N and for long K at N >= 10240, from 65
    at N >= 4096): one ragged 64-row
    tile per 512 columns; first, middle and last column slices against the oracle,
    and a repeated call is bit-identical."""
    assert marlin.plan_2_4(M, K, N)["kernel"] == "large_m"
    assert marlin.plan_2_4(M - 1, K, N)["kernel"] in ("decode", "decode_dma")
    wt, A = _problem(M, N, K, 128, 4100 + M)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    assert torch.equal(_run(wt, A), C), "repeated calls differ"
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2 - 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"prefill M={M} {K}x{N} slice {c0}")


def test_deterministic_repeats():
    """Split-K reductions run in a fixed order: repeated calls are bit-identical
    (the reference's variant smoke test demands identical repeats)."""
    for M, N, K in ((1, 4096, 4096), (16, 1024, 11008), (48, 2048, 4096)):
        wt, A = _problem(M, N, K, 128, 7)
        outs = [_run(wt, A) for _ in range(3)]
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("M", [12, 16])
def test_decode_tail_split(M):
    """Tail split: 4096x22016 has 344 64-column tiles at 9 to 16 rows, 88 past one
    per CU; those 88 are split in two (workgroups 256 + 2 * 88) while the first 256
    run whole. Column slices on both sides of the boundary (chunks 254-257), in the
    middle of the split tiles and at the end match the oracle, and repeated calls
    are bit-identical."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("the tile counts of this case assume 256 CUs")
    p = marlin.plan_2_4(M, 4096, 22016, sms=cus)
    assert p["splits"] == 2 and p["workgroups"] == 256 + 2 * 88
    wt, A = _problem(M, 22016, 4096, 128, 4242 + M)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    for _ in range(3):
        assert torch.equal(_run(wt, A), C), "repeated tail-split calls differ"
    t = to_cpu(wt)
    for c0 in (254, 300, 340):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"tail split M={M} chunks {c0}..{c0 + 3}")


def test_decode_three_tiles_per_workgroup():
    """Llama-2-7B qkv 4096x12288 at 1-4 rows: 768 16-column tiles run three to a
    workgroup of 12 waves (256 workgroups, one per CU), the three sharing the
    workgroup's resident activation rows, in an XCD-ordered tile map of their own.
    Every output column matches the oracle (a tile mapped twice or never shows up as
    a wrong 16-column band), at every M of the padded batches of 1 and 4, with group
    scales; per-column scales on slices; repeats are bit-identical."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("the tile counts of this case assume 256 CUs")
    K, N = 4096, 12288
    for M in (1, 2, 3, 4):
        p = marlin.plan_2_4(M, K, N, sms=cus)
        assert p["kernel"] == "decode" and p["splits"] == 1, (M, p)
        assert p["workgroups"] == 256 and p["threads"] == 768, (M, p)
    wt, A4 = _problem(4, N, K, 128, 5150)
    t = to_cpu(wt)
    ref = oracle_gemm(A4.cpu().numpy(), t)
    for M in (1, 2, 3, 4):
        A = A4[:M].contiguous()
        C = _run(wt, A)
        assert torch.equal(_run(wt, A), C), f"repeated calls differ at M={M}"
        assert_close(C.cpu().numpy(), ref[:M], f"three tiles per workgroup, M={M}")
        # per 16-column tile as well: a misplaced tile is a small share of the columns
        Cn = C.cpu().numpy().astype(np.float64).reshape(M, N // 16, 16)
        rn = ref[:M].astype(np.float64).reshape(M, N // 16, 16)
        err = np.abs(Cn - rn).mean(axis=(0, 2)) / np.abs(rn).mean()
        assert err.max() <= 10 * REL_MAE, f"M={M}: tile {int(err.argmax())} off by {err.max():.3e}"
    wt, A4 = _problem(4, N, K, -1, 5160)
    t = to_cpu(wt)
    for M in (1, 4):
        A = A4[:M].contiguous()
        C = _run(wt, A)
        for c0 in (0, 95, 188):
            r = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
            assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), r, f"g=-1 three tiles M={M} slice {c0}")


@pytest.mark.parametrize("M,K,N,g", [(1, 1024, 12288, 128), (2, 1024, 12288, -1), (4, 512, 12288, 128),
                                     (3, 256, 12288, 128), (1, 1024, 1536, 128), (1, 4096, 1536, -1),
                                     (1, 256, 3072, 128)])
def test_decode_three_tiles_short_k_and_narrow(M, K, N, g):
    """Three tiles per workgroup beyond the 7B qkv shape: short K (fewer than 8
    stages, so the activation rows travel with every stage instead of resident, down
    to a single partial stage at K = 256) and narrow N (1536 / 3072 columns: 32 / 64
    workgroups), grouped and per-column scales; every column against the oracle,
    repeats bit-identical."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus == 256:
        p = marlin.plan_2_4(M, K, N, sms=cus)
        assert p["threads"] == 768 and p["workgroups"] == N // 48 and p["splits"] == 1, p
    wt, A = _problem(M, N, K, g, 7000 + M + K + N)
    C = _run(wt, A)
    assert torch.equal(_run(wt, A), C), "repeated calls differ"
    _check(wt, A, C, f"three tiles M={M} {K}x{N} g={g}")


@pytest.mark.parametrize("M,K,N,splits,wgs", [(1, 4096, 8704, 4, 640), (3, 4096, 8704, 4, 640),
                                             (5, 4096, 4608, 4, 384), (6, 4096, 17408, 4, 640),
                                             (12, 4096, 16896, 4, 288), (16, 2048, 18432, 4, 384)])
def test_decode_tail_split_shapes(M, K, N, splits, wgs):
    """Tail split across the decode kernel's forms: 16-column tiles with resident
    activation rows (M = 1, 3; the XCD chunk remap: 544 tiles, a multiple of 32),
    the 8-row batch on 16-column tiles of 8 waves (M = 5, 288 tiles) and on 32-column
    tiles (M = 6, 544 tiles), 64-column tiles with direct 16-row operands (M = 12,
    16); 32 or 8 tiles past the whole rounds, split four ways. The whole output
    matches the oracle and repeated calls are bit-identical."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("the tile counts of this case assume 256 CUs")
    p = marlin.plan_2_4(M, K, N, sms=cus)
    assert p["splits"] == splits and p["workgroups"] == wgs
    wt, A = _problem(M, N, K, 128, 5150 + M + N)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    assert torch.equal(_run(wt, A), C), "repeated tail-split calls differ"
    _check(wt, A, C, f"tail split M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [(8, 4096, 4096), (2, 4096, 12288), (24, 4096, 22016), (16, 4096, 22016)])
def test_graph_replay_matches_eager(M, K, N):
    """Captured calls replay the eager result bit for bit: 8 rows on 4096x4096 (one
    16-column tile per workgroup, unsplit), 2 rows on 4096x12288 (three 16-column
    tiles per workgroup, resident rows), 24 rows on 4096x22016 (every tile's K
    split in two) and 16 rows on it (only the tail tiles past one round over the CUs
    split), both through the capture stream's scratch, which the eager call on that
    stream made first."""
    if M > 8:
        assert marlin.plan_2_4(M, K, N)["splits"] == 2
    wt, A = _problem(M, N, K, 128, 9)
    ws = torch.zeros(N // 128 * 16, dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C_eager = torch.empty(M, N, dtype=torch.half, device=DEV)
        marlin.mul_2_4(A, wt["B"], wt["meta"], C_eager, wt["s"], ws)
    torch.cuda.synchronize()
    C = torch.zeros(M, N, dtype=torch.half, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(3):
            marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], ws)
    for _ in range(4):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_eager)


@pytest.mark.parametrize("M,K,N,splits", [(256, 4096, 4096, 3), (200, 4096, 8192, 2)])
def test_prefill_graph_replay_split_k(M, K, N, splits):
    """Large-M calls on 64-row tiles split along K (the planner's choice for these
    few-tile shapes; M = 200 leaves a ragged last tile), captured three times in one
    graph on a warmed stream: four replays, each after eager work and a
    synchronisation, equal the eager result bit for bit and the oracle."""
    p = marlin.plan_2_4(M, K, N)
    assert p["kernel"] == "large_m"
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert p["splits"] == splits and p["workgroups"] == splits * (N // 512) * -(-M // 64)
    wt, A = _problem(M, N, K, 128, 77 + M)
    ws = torch.zeros(N // 128 * 16, dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C_eager = torch.empty(M, N, dtype=torch.half, device=DEV)
        marlin.mul_2_4(A, wt["B"], wt["meta"], C_eager, wt["s"], ws)
    torch.cuda.synchronize()
    _check(wt, A, C_eager, f"prefill split-K eager M={M} K={K} N={N}")
    C = torch.zeros(M, N, dtype=torch.half, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(3):
            marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], ws)
    for _ in range(4):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_eager)


def test_layer_forward():
    K, N = 1024, 512
    gen = torch.Generator().manual_seed(3)
    w = (torch.randn((K, N), generator=gen) * 0.02).half().to(DEV)
    q, s, ref = synth.quantize(w, 128)
    layer = marlin.Layer_2_4(K, N, groupsize=128).to(DEV)
    lin = torch.nn.Linear(K, N)
    lin.weight.data = ref
    layer.pack(lin, s, True)
    x = torch.randn((2, 3, K), generator=gen).half().to(DEV)
    y = layer(x)
    assert y.shape == (2, 3, N)
    t = {"B": layer.B.cpu().numpy(), "meta": layer.meta.cpu().numpy(), "s": layer.s.cpu().numpy(),
         "K": K, "N": N, "groupsize": 128, "bits": 4}
    refc = oracle_gemm(x.reshape(6, K).cpu().numpy(), t)
    assert_close(y.reshape(6, N).cpu().numpy(), refc, "Layer_2_4.forward")


def test_kernel_shape_errors_raise():
    wt, A = _problem(32, 512, 1024, -1, 5)
    with pytest.raises(RuntimeError, match="No kernel implementation for thread_k=128, thread_m=128"):
        _run(wt, A, thread_k=128, thread_m=128)
    with pytest.raises(RuntimeError, match=r"Problem \(m=512, n=32, k=1024\) not compatible"):
        _run(wt, A, thread_k=64, thread_m=384)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 12288), (16, 11008, 4096), (64, 4096, 22016), (512, 8192, 8192)])
def test_per_column_scales_full_size(M, K, N):
    """Group size -1 (one scale per output column, applied after the fp16 round of the
    sum, marlin_cuda_kernel_nm.cu:579-585) on every kernel at full Llama sizes: the
    decode kernel, chunked decode launches and the large-M kernel."""
    wt, A = _problem(M, N, K, -1, 31 + M)
    C = _run(wt, A)
    assert torch.isfinite(C).all()
    assert torch.equal(_run(wt, A), C), "repeated calls differ"
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2 - 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"g=-1 {K}x{N} M={M} slice {c0}")
