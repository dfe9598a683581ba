"""GPU parity of the 3-bit variants: the 3-bit metadata codec and GEMM (reference
metadata_decode experiment), the 3-bit code expansion (3bit_encoding experiment),
and the 3-bit nonzero-value GEMM of benchmark config 4."""
import numpy as np
import pytest
import torch

from csed499ii_amd import marlin, synth
from oracle import sm24_oracle as o
from tests.gpu_util import assert_close, oracle_gemm, slice_cols, to_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ws(N):
    return torch.zeros(max(N // 128 * 16, 16), dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("K,N", [(1024, 512), (4096, 4096)])
def test_meta3_codec_bit_exact(K, N):
    wt = synth.make_weight(K, N, 5, 128, device=DEV)
    packed = marlin.pack_meta3(wt["meta"].reshape(-1))
    ref, bad = o.meta3_pack(wt["meta"].cpu().numpy())
    assert bad == 0
    assert packed.numel() == wt["meta"].numel() * 3 // 8
    assert np.array_equal(packed.cpu().numpy().view(np.uint32), ref)
    back = marlin.unpack_meta3(packed)
    assert torch.equal(back, wt["meta"].reshape(-1))


def test_meta3_rejects_invalid_nibbles():
    meta = torch.full((256,), 0x4444, dtype=torch.int16, device=DEV)
    meta[17] = 0x4443
    with pytest.raises(RuntimeError, match="unsupported 2:4 nibbles"):
        marlin.pack_meta3(meta)


@pytest.mark.parametrize("M,N,K,g", [(1, 4096, 4096, 128), (16, 4096, 4096, 128), (48, 1024, 2048, -1),
                                     (16, 12288, 4096, 128), (32, 4096, 4096, 128), (20, 12288, 4096, -1),
                                     (300, 1024, 1024, 128), (512, 4096, 4096, -1)])
def test_meta3_gemm_equals_baseline_bit_exact(M, N, K, g):
    """Same arithmetic, compressed metadata: outputs must be identical."""
    wt = synth.make_weight(K, N, M + N, g, device=DEV)
    A = synth.make_activation(M, K, 3, device=DEV)
    packed = marlin.pack_meta3(wt["meta"].reshape(-1))
    C0 = torch.empty(M, N, dtype=torch.half, device=DEV)
    C1 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C0, wt["s"], _ws(N))
    marlin.mul_2_4_meta3(A, wt["B"], packed, C1, wt["s"], _ws(N))
    torch.cuda.synchronize()
    assert torch.equal(C0, C1)
    if N <= 4096:
        assert_close(C1.cpu().numpy(), oracle_gemm(A.cpu().numpy(), to_cpu(wt)), "meta3")


@pytest.mark.parametrize("M", [1, 16, 32, 256])
@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 12288), (4096, 22016), (11008, 4096)])
def test_w3_gemm_config4(M, K, N):
    """Benchmark config 4: 3-bit values, Llama-2-7B shapes, M in {1, 16, 256}."""
    wt = synth.make_weight(K, N, 4 + K + N, 128, bits=3, device=DEV)
    A = synth.make_activation(M, K, 4, device=DEV)
    C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4_w3(A, wt["B"], wt["meta"], C, wt["s"], _ws(N))
    torch.cuda.synchronize()
    assert torch.isfinite(C).all()
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"w3 {K}x{N} M={M} slice {c0}")


def test_w3_gemm_small_full_oracle():
    # (K=192 needs the reference's 64-deep tile: the automatic 128-deep tile rejects it)
    for M, N, K, g, tk, tm in ((5, 512, 1024, -1, -1, -1), (16, 768, 192, -1, 64, 256),
                               (33, 1024, 2048, 128, -1, -1)):
        wt = synth.make_weight(K, N, M, g, bits=3, device=DEV)
        A = synth.make_activation(M, K, M, device=DEV)
        C = torch.empty(M, N, dtype=torch.half, device=DEV)
        marlin.mul_2_4_w3(A, wt["B"], wt["meta"], C, wt["s"], _ws(N), tk, tm)
        torch.cuda.synchronize()
        assert_close(C.cpu().numpy(), oracle_gemm(A.cpu().numpy(), to_cpu(wt)), f"w3 {M}x{N}x{K}")


def test_expand3_exhaustive():
    """All 2^24 packed 8-code inputs (3bit_encoding/experiment.cu:70, 84)."""
    x = np.arange(1 << 24, dtype=np.uint32)
    stream = np.stack([x & 255, (x >> 8) & 255, (x >> 16) & 255], axis=-1).astype(np.uint8).ravel()
    got = marlin.expand3(torch.from_numpy(stream).to(DEV))
    torch.cuda.synchronize()
    ref = o.expand3(stream)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref)


@pytest.mark.parametrize("groups", [1, 2, 3, 7, 9, 31, 33])
def test_expand3_partial_blocks(groups):
    """Group counts that leave partial thread blocks (experiment.cu:87)."""
    rng = np.random.default_rng(groups)
    stream = rng.integers(0, 256, size=48 * groups, dtype=np.uint8)
    got = marlin.expand3(torch.from_numpy(stream).to(DEV))
    assert np.array_equal(got.cpu().numpy().view(np.uint32), o.expand3(stream))


def _w3_as_w4(B3: torch.Tensor) -> torch.Tensor:
    """The 4-bit packed words holding the same values as a 3-bit value stream: word w
    is the 24-bit field at byte 3w, code p at bits 3p, moved to nibble p with the
    zero point 4 -> 8 (restated on the CPU from the 3-bit layout, for this test)."""
    b = B3.cpu().numpy().view(np.uint8).reshape(-1, 3).astype(np.uint32)
    f = b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)
    w = np.zeros_like(f)
    for p in range(8):
        w |= (((f >> (3 * p)) & 7) + 4) << (4 * p)
    return torch.from_numpy(w.view(np.int32).copy()).to(DEV)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (16, 4096, 4096), (32, 1024, 8192), (256, 4096, 4096),
                                   (300, 1024, 8192)])
def test_w3_gemm_bit_exact_against_4bit_path(M, K, N):
    """3-bit values give exactly the products of the same values packed at 4 bits
    ((code - 4) * s == (nibble - 8) * s in fp16), on the decode kernel and on the
    large-M path that expands them first: the outputs are bit-identical."""
    wt = synth.make_weight(K, N, 7 + K + M, 128, bits=3, device=DEV)
    A = synth.make_activation(M, K, 9, device=DEV)
    B4 = _w3_as_w4(wt["B"])
    C3 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    C4 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4_w3(A, wt["B"], wt["meta"], C3, wt["s"], _ws(N))
    marlin.mul_2_4(A, B4, wt["meta"], C4, wt["s"], _ws(N))
    torch.cuda.synchronize()
    assert torch.isfinite(C3).all()
    assert torch.equal(C3, C4)


# Shapes that the decode tile table sends to the 8-row batch at 5-8 rows (activations
# staged through LDS): 4096x4096 on 16-column tiles of 8 waves, 4096x22016 at M = 5 on
# 32-column tiles, 8192x57344 on 64-column tiles.
MB8_CASES = [(5, 4096, 4096), (8, 4096, 4096), (5, 4096, 22016), (5, 8192, 57344), (8, 8192, 57344)]


@pytest.mark.parametrize("M,K,N", MB8_CASES)
def test_8row_batch_w3(M, K, N):
    """3-bit values on the 8-row batch: oracle column slices, and bit-identical to the
    same values packed at 4 bits."""
    wt = synth.make_weight(K, N, 11 + K + M, 128, bits=3, device=DEV)
    A = synth.make_activation(M, K, 13 + M, device=DEV)
    C3 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    C4 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4_w3(A, wt["B"], wt["meta"], C3, wt["s"], _ws(N))
    marlin.mul_2_4(A, _w3_as_w4(wt["B"]), wt["meta"], C4, wt["s"], _ws(N))
    torch.cuda.synchronize()
    assert torch.equal(C3, C4)
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C3[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"w3 {K}x{N} M={M} slice {c0}")


@pytest.mark.parametrize("M,K,N", MB8_CASES)
def test_8row_batch_meta3(M, K, N):
    """3-bit metadata on the 8-row batch: bit-identical to the 4-bit metadata call and
    equal to the oracle on column slices."""
    wt = synth.make_weight(K, N, 17 + K + M, 128, device=DEV)
    A = synth.make_activation(M, K, 19 + M, device=DEV)
    C0 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    C1 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C0, wt["s"], _ws(N))
    marlin.mul_2_4_meta3(A, wt["B"], marlin.pack_meta3(wt["meta"].reshape(-1)), C1, wt["s"], _ws(N))
    torch.cuda.synchronize()
    assert torch.equal(C0, C1)
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C1[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"meta3 {K}x{N} M={M} slice {c0}")


@pytest.mark.parametrize("M,K,N", MB8_CASES)
def test_8row_batch_per_column_scales(M, K, N):
    """Per-column scales (groupsize -1: the scale multiplies the fp16-rounded output)
    on the 8-row batch, against the oracle on column slices."""
    wt = synth.make_weight(K, N, 23 + K + M, -1, device=DEV)
    A = synth.make_activation(M, K, 29 + M, device=DEV)
    C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], _ws(N))
    torch.cuda.synchronize()
    t = to_cpu(wt)
    chunks = N // 64
    for c0 in (0, chunks // 2, chunks - 4):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"g=-1 {K}x{N} M={M} slice {c0}")


@pytest.mark.parametrize("M,K", [(1, 4096), (2, 4096), (4, 4096), (1, 1024), (4, 512)])
def test_three_tiles_per_workgroup_3bit_paths(M, K):
    """Llama-2-7B qkv 4096x12288 at 1-4 rows runs three 16-column tiles per workgroup
    of 12 waves with 3-bit values and with 3-bit metadata as with 4-bit operands
    (and at K = 512 / 1024, where the activation rows travel with every stage):
    both are bit-identical to the 4-bit call on the same values, which the oracle
    checks on column slices."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("the tile counts of this case assume 256 CUs")
    N = 12288
    p = marlin.plan_2_4(M, K, N, sms=cus)
    assert p["workgroups"] == 256 and p["threads"] == 768, p
    wt = synth.make_weight(K, N, 23 + M + K, 128, bits=3, device=DEV)
    A = synth.make_activation(M, K, 29 + M, device=DEV)
    C3 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    C4 = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    Cm = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    B4 = _w3_as_w4(wt["B"])
    marlin.mul_2_4_w3(A, wt["B"], wt["meta"], C3, wt["s"], _ws(N))
    marlin.mul_2_4(A, B4, wt["meta"], C4, wt["s"], _ws(N))
    marlin.mul_2_4_meta3(A, B4, marlin.pack_meta3(wt["meta"].reshape(-1)), Cm, wt["s"], _ws(N))
    torch.cuda.synchronize()
    assert torch.equal(C3, C4), "3-bit values differ from the 4-bit call"
    assert torch.equal(Cm, C4), "3-bit metadata differs from the 4-bit call"
    t = to_cpu(wt)
    for c0 in (0, 95, 188):
        ref = oracle_gemm(A.cpu().numpy(), slice_cols(t, c0, 4))
        assert_close(C3[:, 64 * c0:64 * (c0 + 4)].cpu().numpy(), ref, f"w3 three tiles M={M} slice {c0}")
