"""Host-side product code (torch, CPU) against the oracle and the reference's
golden vectors: converters, permutations, pack(), Layer_2_4, replace_linear."""
import numpy as np
import pytest
import torch
import torch.nn as nn

from csed499ii_amd import marlin, synth
from csed499ii_amd.marlin import _semi_structured_conversions as sc
from oracle import sm24_oracle as o

GOLD = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "semi_structured.npz")


@pytest.mark.parametrize("tag", ["a", "b", "c", "d"])
def test_converter_matches_reference_vectors(tag):
    dense = torch.from_numpy(GOLD[f"conv_{tag}_dense"])
    sparse, meta = sc.sparse_semi_structured_from_dense_cutlass(dense)
    assert np.array_equal(sparse.numpy(), GOLD[f"conv_{tag}_sparse"])
    assert np.array_equal(meta.numpy(), GOLD[f"conv_{tag}_meta"])
    back = sc.sparse_semi_structured_to_dense_cutlass(torch.from_numpy(GOLD[f"conv_{tag}_sparse"]),
                                                       torch.from_numpy(GOLD[f"conv_{tag}_meta"]))
    assert np.array_equal(back.numpy(), GOLD[f"conv_{tag}_back"])


def test_converter_half_matches_reference_vectors():
    sparse, meta = sc.sparse_semi_structured_from_dense_cutlass(torch.from_numpy(GOLD["conv_h_dense"]))
    assert np.array_equal(sparse.numpy(), GOLD["conv_h_sparse"])
    assert np.array_equal(meta.numpy(), GOLD["conv_h_meta"])


def test_converter_boolean_encoding_matches_table():
    """The product's boolean encoder against the 16-row table of the reference comments."""
    for flags, code in o.META_TABLE.items():
        f = [torch.tensor([bool(x)]) for x in flags]
        i0, i1 = sc._encode_groups(*f)
        assert (int(i0) | int(i1) << 2) == code


def test_converter_errors():
    with pytest.raises(RuntimeError, match="2-dimensional"):
        sc.sparse_semi_structured_from_dense_cutlass(torch.zeros(64))
    with pytest.raises(RuntimeError, match="divisible by 32"):
        sc.sparse_semi_structured_from_dense_cutlass(torch.zeros(48, 32, dtype=torch.half))
    with pytest.raises(RuntimeError, match="divisible by 16"):
        sc.sparse_semi_structured_from_dense_cutlass(torch.zeros(64, 24, dtype=torch.half))
    with pytest.raises(RuntimeError, match="Invalid datatype"):
        sc.sparse_semi_structured_from_dense_cutlass(torch.zeros(64, 32, dtype=torch.float64))
    with pytest.raises(RuntimeError, match="meta matrix"):
        sc.sparse_semi_structured_to_dense_cutlass(torch.zeros(64, 16, dtype=torch.half),
                                                   torch.zeros(32, 2, dtype=torch.int16))


def test_mask_creator_matches_reference_on_tie_free_vectors():
    assert np.array_equal(sc.mask_creator(torch.from_numpy(GOLD["mask_x"])).numpy(), GOLD["mask_ref"])


def test_mask_creator_ties_keep_lower_index():
    x = torch.tensor([[1.0, 1.0, 1.0, 1.0], [0.0, 2.0, 2.0, 2.0], [3.0, -3.0, 0.0, 3.0]])
    m = sc.mask_creator(x)
    assert m.tolist() == [[1, 1, 0, 0], [0, 1, 1, 0], [1, 1, 0, 0]]
    assert np.array_equal(m.numpy().astype(bool), o.mask_2_4(x.numpy(), axis=-1))


def test_perms_match_oracle():
    perm, scale_perm, scale_perm_single = o.get_perms_2_4()
    assert np.array_equal(marlin._perm_2_4.numpy(), perm)
    assert marlin._scale_perm_2_4 == scale_perm.tolist()
    assert marlin._scale_perm_single_2_4 == scale_perm_single.tolist()


@pytest.mark.parametrize("K,N,g", [(128, 64, 128), (256, 128, -1), (512, 256, 128), (1024, 512, -1)])
def test_pack_reference_rule_matches_oracle(K, N, g):
    gen = torch.Generator().manual_seed(K * 7 + N)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    q, s, ref = synth.quantize(w, g)
    B, sp, meta = marlin.pack_2_4(ref, s, g)
    Bo, spo, metao = o.pack(ref.numpy(), s.numpy(), g)
    assert B.shape == (K // 32, 2 * N) and B.dtype == torch.int32
    assert meta.shape == (N, K // 16) and meta.dtype == torch.int16
    assert np.array_equal(B.numpy(), Bo)
    assert np.array_equal(sp.numpy(), spo)
    assert np.array_equal(meta.numpy(), metao)


@pytest.mark.parametrize("K,N,g", [(128, 64, 128), (512, 256, 128), (1024, 512, -1)])
def test_pack_explicit_mask_matches_oracle(K, N, g):
    gen = torch.Generator().manual_seed(K + 3 * N)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    mask = synth.prune_2_4(w)
    w = w * mask
    assert np.array_equal(mask.numpy(), o.mask_2_4(w.numpy(), axis=0))
    q, s, ref = synth.quantize(w, g)
    B, sp, meta = marlin.pack_2_4(w, s, g, mask=mask)
    Bo, spo, metao = o.pack(w.numpy(), s.numpy(), g, mask=mask.numpy())
    assert np.array_equal(B.numpy(), Bo)
    assert np.array_equal(sp.numpy(), spo)
    assert np.array_equal(meta.numpy(), metao)
    # the packed operands dequantize to exactly the quantizer's reference weight
    W = o.dequant(Bo, metao, spo, K, N, g)
    assert np.array_equal(W, (ref * mask).numpy())


def test_pack_w3_matches_oracle():
    K, N, g = 512, 256, 128
    gen = torch.Generator().manual_seed(77)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    mask = synth.prune_2_4(w)
    w = w * mask
    q, s, ref = synth.quantize(w, g, maxq=7)
    assert q.max() <= 7
    B3, sp, meta = marlin.pack_w3(w, s, g, mask)
    B3o, spo, metao = o.pack_w3(w.numpy(), s.numpy(), g, mask.numpy())
    assert B3.dtype == torch.uint8 and B3.numel() == K * N * 3 // 16
    assert np.array_equal(B3.numpy(), B3o)
    assert np.array_equal(meta.numpy(), metao)
    assert np.array_equal(o.dequant_w3(B3o, metao, spo, K, N, g), (ref * mask).numpy())


def test_quantizer_matches_oracle():
    gen = torch.Generator().manual_seed(5)
    w = (torch.randn((512, 128), generator=gen) * 0.02).half()
    for g, maxq in ((128, 15), (-1, 15), (128, 7)):
        q, s, ref = synth.quantize(w, g, maxq)
        qo, so, refo = o.quantize(w.numpy(), g, maxq)
        assert np.array_equal(q.numpy(), qo)
        assert np.array_equal(s.numpy(), so)
        assert np.array_equal(ref.numpy(), refo)


def test_layer_pack_buffers_and_state_dict():
    K, N = 256, 128
    layer = marlin.Layer_2_4(K, N, groupsize=128)
    assert layer.B.shape == (K // 32, 2 * N)
    gen = torch.Generator().manual_seed(1)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    q, s, ref = synth.quantize(w, 128)
    lin = nn.Linear(K, N)
    lin.weight.data = ref  # read as K x N, as the reference does
    layer.pack(lin, s, True)
    Bo, spo, metao = o.pack(ref.numpy(), s.numpy(), 128)
    assert np.array_equal(layer.B.numpy(), Bo)
    assert np.array_equal(layer.s.numpy(), spo)
    assert np.array_equal(layer.meta.numpy(), metao)
    assert layer.k == K and layer.groupsize == 128  # pack is idempotent here
    sd = layer.state_dict()
    assert set(sd) == {"B", "meta", "s"}
    layer2 = marlin.Layer_2_4(K, N, groupsize=128)
    layer2.load_state_dict(sd)
    assert torch.equal(layer2.B, layer.B)


def test_layer_errors():
    with pytest.raises(ValueError, match="groupsize"):
        marlin.Layer_2_4(256, 128, groupsize=64)
    with pytest.raises(ValueError, match="divisible"):
        marlin.Layer_2_4(200, 128)
    layer = marlin.Layer_2_4(256, 128)
    lin = nn.Linear(256, 128)
    with pytest.raises(ValueError, match="half"):
        layer.pack(lin, torch.ones(1, 128, dtype=torch.half), True)
    lin.weight.data = torch.zeros(256, 128, dtype=torch.half)
    with pytest.raises(ValueError, match="trans=False"):
        layer.pack(lin, torch.ones(1, 128, dtype=torch.half))


def test_replace_linear():
    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.q = nn.Linear(256, 128)
            self.o = nn.Linear(128, 256)
            self.sub = nn.Sequential(nn.Linear(256, 256), nn.ReLU())
            self.inner = nn.Module()
            self.inner.proj = nn.Linear(256, 256)

    m = Block()
    marlin.replace_linear(m, name_filter=lambda n: n != "o", groupsize=128)
    assert isinstance(m.q, marlin.Layer_2_4)
    assert isinstance(m.o, nn.Linear)
    assert isinstance(m.inner.proj, marlin.Layer_2_4)
    # as in the reference, attribute discovery uses dir(), which omits the numeric
    # child names of containers such as nn.Sequential
    assert isinstance(m.sub[0], nn.Linear)
    assert (m.q.k, m.q.n, m.q.groupsize) == (256, 128, 128)


def test_mul_2_4_binding_checks_on_cpu():
    """Shape inference and the reference binding's messages (marlin_cuda.cpp:74-80)
    fire before any device work."""
    A = torch.zeros(16, 256, dtype=torch.half)
    C = torch.zeros(16, 128, dtype=torch.half)
    B = torch.zeros(256 * 128 // 16, dtype=torch.int32)
    meta = torch.zeros(256 * 128 // 16, dtype=torch.int16)
    ws = torch.zeros(128 // 128 * 16, dtype=torch.int32)
    with pytest.raises(RuntimeError, match=r"k=256 not compatible with 3 groups\."):
        marlin.mul_2_4(A, B, meta, C, torch.zeros(3, 128, dtype=torch.half), ws)
    with pytest.raises(RuntimeError, match=r"workspace must be of size at least 16\."):
        marlin.mul_2_4(A, B, meta, C, torch.zeros(2, 128, dtype=torch.half), ws[:8])
    with pytest.raises(RuntimeError, match="GPU tensor"):
        marlin.mul_2_4(A, B, meta, C, torch.zeros(2, 128, dtype=torch.half), ws)


# ---- dense Marlin packing (reference __init__.py:134-226) ----


@pytest.mark.parametrize("K,N,g", [(128, 256, 128), (256, 512, -1), (1024, 768, 128), (512, 256, -1)])
def test_pack_dense_matches_oracle(K, N, g):
    """The product's closed-form placement equals the oracle's restated permutation
    (reference __init__.py:78-99, 213-223), codes and scales bit-exact."""
    gen = torch.Generator().manual_seed(K + 3 * N)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    _, s, _ = synth.quantize(w, g)
    B, sp = marlin.pack_dense(w, s, g)
    Bo, spo = o.dense_pack(w.numpy(), s.numpy(), g)
    assert B.shape == (K // 16, 2 * N) and B.dtype == torch.int32
    assert np.array_equal(B.numpy(), Bo)
    assert np.array_equal(sp.numpy().view(np.int16), np.asarray(spo, np.float16).view(np.int16))


def test_dense_layer_pack_and_checks():
    K, N = 256, 512
    gen = torch.Generator().manual_seed(9)
    w = (torch.randn((K, N), generator=gen) * 0.02).half()
    _, s, ref = synth.quantize(w, 128)
    layer = marlin.Layer(K, N, groupsize=128)
    lin = nn.Linear(K, N)
    lin.weight.data = ref  # read as K x N, as the reference does
    layer.pack(lin, s)
    Bo, spo = o.dense_pack(ref.numpy(), s.numpy(), 128)
    assert np.array_equal(layer.B.numpy(), Bo)
    assert set(layer.state_dict()) == {"B", "s"}
    with pytest.raises(ValueError, match="transposed"):
        layer.pack(lin, s, trans=True)
    with pytest.raises(ValueError, match="divisible"):
        marlin.Layer(K, 320)
    with pytest.raises(ValueError, match="groupsize"):
        marlin.Layer(K, N, groupsize=64)
