"""GPU parity of the lane-native decode layout: the repack and its inverse against
the oracle (bit-exact), and the GEMM on it against the CPU oracle of the original
weight (the layout is this library's own; the reference has no counterpart)."""
import numpy as np
import pytest
import torch

from csed499ii_amd import marlin, synth
from oracle import sm24_oracle as o
from tests.gpu_util import assert_close, oracle_gemm, slice_cols, to_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("K,N,g", [(256, 64, 128), (512, 128, -1), (1024, 512, 128), (4096, 4096, 128)])
def test_native_pack_and_unpack_bit_exact(K, N, g):
    wt = synth.make_weight(K, N, 31 + K, g, device=DEV)
    Bn, Mn, Sn = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    torch.cuda.synchronize()
    t = to_cpu(wt)
    W_ref, X_ref, S_ref = o.native_pack(t["B"], t["meta"], t["s"], K, N, g)
    assert np.array_equal(Bn.cpu().numpy().view(np.uint32), W_ref)
    assert np.array_equal(Mn.cpu().numpy().view(np.uint16), X_ref)
    assert np.array_equal(Sn.cpu().numpy().view(np.uint16), np.asarray(S_ref, np.float16).view(np.uint16))
    B, meta, s = marlin.unpack_native(Bn, Mn, Sn)
    torch.cuda.synchronize()
    assert torch.equal(B.reshape(-1), wt["B"].reshape(-1))
    assert torch.equal(meta.reshape(-1), wt["meta"].reshape(-1))
    assert torch.equal(s.view(torch.int16).reshape(-1), wt["s"].view(torch.int16).reshape(-1))


def _native_run(A, nat, N):
    C = torch.full((A.shape[0], N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4_native(A, *nat[:2], C, nat[2])
    torch.cuda.synchronize()
    return C


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 13, 16, 17, 32])
@pytest.mark.parametrize("K,N,g", [(256, 128, 128), (1024, 512, -1), (2048, 1024, 128)])
def test_native_gemm_full_oracle(M, K, N, g):
    """M <= 16: the native kernel (1, 4, 8 or 16 staged batch rows); M > 16: unpack
    into the staging buffer and the reference-layout kernels, whose tiles need
    N % 256 == 0 above 16 rows."""
    wt = synth.make_weight(K, N, 7 * M + K, g, device=DEV)
    A = synth.make_activation(M, K, 11 + M, device=DEV)
    nat = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    if M > 16 and N % 256:
        with pytest.raises(RuntimeError, match="not compatible"):
            _native_run(A, nat, N)
        return
    C = _native_run(A, nat, N)
    assert_close(C.cpu().numpy(), oracle_gemm(A.cpu().numpy(), to_cpu(wt)), f"native {M}x{N}x{K} g={g}")
    assert torch.equal(_native_run(A, nat, N), C), "repeated calls differ"


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("K,N", [(4096, 12288), (11008, 4096), (8192, 8192), (28672, 8192)])
def test_native_gemm_full_size_slices(K, N, M):
    """Llama-2-7B/70B decode shapes.  The native planner splits K in two at M = 4 from
    K = 16384 (28672x8192), and at 8-16 rows when the widest tile's workgroups cover
    less than 60 % of the CUs (11008x4096 and 28672x8192 at M = 8, 16); M = 1 never
    splits.  Checked on column slices against the oracle and whole against mul_2_4
    on the original weight; repeated calls bit-identical (split-K hand-off in split
    order)."""
    wt = synth.make_weight(K, N, K + N + M, 128, device=DEV)
    A = synth.make_activation(M, K, 3 + M, device=DEV)
    nat = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    C = _native_run(A, nat, N)
    assert torch.isfinite(C).all()
    for _ in range(3):
        assert torch.equal(_native_run(A, nat, N), C), "repeated calls differ"
    C_ref = torch.empty_like(C)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C_ref, wt["s"], torch.zeros(N // 128 * 16, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert_close(C.cpu().numpy(), C_ref.cpu().numpy(), f"native vs mul_2_4 {K}x{N} M={M}")
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2 - 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"native {K}x{N} M={M} slice {c0}")


def test_native_rejects_bad_shapes():
    wt = synth.make_weight(384, 128, 5, 128, device=DEV)  # K % 256 != 0
    with pytest.raises(RuntimeError, match="K % 256"):
        marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    # N = 64 serves M <= 16 natively; larger batches follow mul_2_4's tile rules
    wt = synth.make_weight(256, 64, 6, 128, device=DEV)
    nat = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    for m in (4, 16):
        A = synth.make_activation(m, 256, 6, device=DEV)
        C = _native_run(A, nat, 64)
        assert_close(C.cpu().numpy(), oracle_gemm(A.cpu().numpy(), to_cpu(wt)), f"native N=64 M={m}")
    with pytest.raises(RuntimeError, match="not compatible"):
        _native_run(synth.make_activation(17, 256, 6, device=DEV), nat, 64)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (16, 11008, 4096), (4, 28672, 8192)])
def test_native_graph_replay_matches_eager(M, K, N):
    """Captured native calls replay the eager result bit for bit, with eager work and
    synchronisations between the replays: one unsplit shape and two that split K
    (11008x4096 at M = 16 four ways, 28672x8192 at M = 4 in two).  The eager call
    runs first on the capture stream, so that stream already has its split-K
    scratch and the captured calls split as the eager one did."""
    wt = synth.make_weight(K, N, 77 + M, 128, device=DEV)
    A = synth.make_activation(M, K, 78, device=DEV)
    nat = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C_eager = _native_run(A, nat, N)
    C = torch.zeros(M, N, dtype=torch.half, device=DEV)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(3):
            marlin.mul_2_4_native(A, *nat[:2], C, nat[2])
    for _ in range(4):
        C.fill_(float("nan"))
        assert torch.equal(_native_run(A, nat, N), C_eager)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, C_eager)


@pytest.mark.parametrize("M", [8, 16])
def test_native_gemm_two_block_tiles(M):
    """K = 4096, N = 8192 at 8 and 16 rows: the native planner's two-block tiles (four
    blocks leave too few workgroups, 128 on 256 CUs, and K = 4096 is too short to
    split), against the oracle on column slices and against mul_2_4 whole."""
    K, N = 4096, 8192
    wt = synth.make_weight(K, N, 41 + M, 128, device=DEV)
    A = synth.make_activation(M, K, 42 + M, device=DEV)
    nat = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    C = _native_run(A, nat, N)
    assert torch.equal(_native_run(A, nat, N), C), "repeated calls differ"
    C_ref = torch.empty_like(C)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C_ref, wt["s"], torch.zeros(N // 128 * 16, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert_close(C.cpu().numpy(), C_ref.cpu().numpy(), f"native vs mul_2_4 {K}x{N} M={M}")
    t = to_cpu(wt)
    for c0 in (0, 62, 124):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"native {K}x{N} M={M} slice {c0}")


def test_layer_to_native():
    """Layer_2_4.to_native: batches of <= 16 rows run on the native copy, larger ones
    on the pack() buffers; the state_dict keeps only the pack() buffers; a later
    pack() refreshes the copy."""
    K, N = 1024, 512
    gen = torch.Generator().manual_seed(12)
    w = (torch.randn((K, N), generator=gen) * 0.02).half().to(DEV)
    q, s, ref = synth.quantize(w, 128)
    lin = torch.nn.Linear(K, N)
    lin.weight.data = ref
    layer = marlin.Layer_2_4(K, N, groupsize=128).to(DEV)
    layer.pack(lin, s, True)
    t = {"B": layer.B.cpu().numpy(), "meta": layer.meta.cpu().numpy(), "s": layer.s.cpu().numpy(),
         "K": K, "N": N, "groupsize": 128, "bits": 4}
    keys = set(layer.state_dict())
    assert layer.to_native() is layer
    assert set(layer.state_dict()) == keys
    for rows in (1, 3, 8, 16, 40):
        x = torch.randn((rows, K), generator=gen).half().to(DEV)
        y = layer(x)
        torch.cuda.synchronize()
        assert_close(y.cpu().numpy(), oracle_gemm(x.cpu().numpy(), t), f"Layer_2_4 native rows={rows}")
    lin.weight.data = (ref * 2).half()
    layer.pack(lin, (s * 2).half(), True)
    t2 = {"B": layer.B.cpu().numpy(), "meta": layer.meta.cpu().numpy(), "s": layer.s.cpu().numpy(),
          "K": K, "N": N, "groupsize": 128, "bits": 4}
    x = torch.randn((2, K), generator=gen).half().to(DEV)
    assert_close(layer(x).cpu().numpy(), oracle_gemm(x.cpu().numpy(), t2), "Layer_2_4 native after re-pack")


@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_native_per_column_scales_full_size(M):
    """Group size -1 on the native layout at a Llama-2-7B shape (scales applied after
    the fp16 round of the sum, as on the pack() layout)."""
    K, N = 4096, 12288
    wt = synth.make_weight(K, N, 41 + M, -1, device=DEV)
    A = synth.make_activation(M, K, 42, device=DEV)
    nat = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
    assert nat[2].shape == (1, N)
    C = _native_run(A, nat, N)
    t = to_cpu(wt)
    for c0 in (0, 95, 188):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"native g=-1 M={M} slice {c0}")
