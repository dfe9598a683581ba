"""The caller side of the op end to end: a synthetic 32-layer
Llama-2-7B-shaped model whose nn.Linear layers ``replace_linear`` turns into
``Layer_2_4`` (reference marlin/__init__.py:391-415), packed layer by layer with
``Layer_2_4.pack`` (274-388) and put on the lane-native layout with ``to_native()``.
Its forward for M in {1, 8, 32} is captured in one HIP graph; every linear's output
is checked on a column slice against the CPU oracle of that linear's packed weight
and actual input.  A ``state_dict`` saved and loaded into a fresh replace_linear'd
model reproduces the outputs bit for bit."""
import io

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from csed499ii_amd import marlin, synth
from tests.gpu_util import assert_close, oracle_gemm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LAYERS = 32
HID, FFN = 4096, 11008
MS = (1, 8, 32)


def _rms(x):
    """RMS normalisation (Llama's input and post-attention norms, without weights):
    keeps the fp16 residual stream of the synthetic stack in range."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).half()


class Block(nn.Module):
    """One Llama-2-7B-shaped layer: fused QKV, O, fused gate/up and down projections.
    The attention is a stand-in (the q third of QKV feeds O); every linear's input and
    output are appended to ``trace``."""

    def __init__(self):
        super().__init__()
        self.qkv = nn.Linear(HID, 3 * HID, bias=False)
        self.o = nn.Linear(HID, HID, bias=False)
        self.gate_up = nn.Linear(HID, 2 * FFN, bias=False)
        self.down = nn.Linear(FFN, HID, bias=False)

    def forward(self, x, trace):
        def lin(name, inp):
            out = getattr(self, name)(inp)
            trace.append((name, inp, out))
            return out

        h = lin("qkv", _rms(x))
        x = x + 0.5 * lin("o", h[:, :HID].contiguous())
        gu = lin("gate_up", _rms(x))
        m = (F.silu(gu[:, :FFN].float()) * gu[:, FFN:].float()).half()
        return x + 0.5 * lin("down", m)


class Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([Block() for _ in range(LAYERS)])

    def forward(self, x, trace):
        for blk in self.layers:
            x = blk(x, trace)
        return x


def _empty_model():
    """nn.Linear weights on the meta device (never materialised), then
    replace_linear: empty Layer_2_4 buffers on the GPU."""
    with torch.device("meta"):
        model = Model()
    with torch.device(DEV):
        marlin.replace_linear(model, groupsize=128)
    return model


class _Lin:
    """What Layer_2_4.pack reads: ``.weight`` as K x N (reference __init__.py:349)."""

    def __init__(self, w):
        self.weight = nn.Parameter(w, requires_grad=False)


def _pack_model(model):
    gen = torch.Generator(device=DEV).manual_seed(20261019 + 5)
    for blk in model.layers:
        for name in ("qkv", "o", "gate_up", "down"):
            layer = getattr(blk, name)
            w = (torch.randn((layer.k, layer.n), device=DEV, generator=gen) * 0.02).half()
            mask = synth.prune_2_4(w)
            w = w * mask
            _, s, _ = synth.quantize(w, 128)
            layer.pack(_Lin(w), s, True, mask=mask)
            del w, mask
    torch.cuda.synchronize()
    return model


def _slice_packed(layer, c0, nc):
    """Columns [64 c0, 64 (c0 + nc)) of a packed Layer_2_4, sliced on the GPU, as the
    host dict the oracle reads."""
    K, N = layer.k, layer.n
    t = {"B": layer.B.reshape(K // 32, 2 * N)[:, 128 * c0:128 * (c0 + nc)].cpu().numpy(),
         "meta": layer.meta.reshape(K // 32, 2 * N)[:, 128 * c0:128 * (c0 + nc)].cpu().numpy(),
         "s": layer.s[:, 64 * c0:64 * (c0 + nc)].cpu().numpy(), "K": K, "N": 64 * nc, "groupsize": 128,
         "bits": 4}
    return t


def _natives(model):
    """to_native() on every layer; its repacks run on the current stream, so wait for
    them before another stream reads the copies."""
    for mod in model.modules():
        if isinstance(mod, marlin.Layer_2_4):
            mod.to_native()
    torch.cuda.synchronize()
    return model


@pytest.fixture(scope="module")
def model():
    return _natives(_pack_model(_empty_model()))


def _inputs():
    """Activations for every M, complete before any other stream reads them."""
    gen = torch.Generator(device=DEV).manual_seed(77)
    xs = {M: torch.randn((M, HID), device=DEV, generator=gen).half() for M in MS}
    torch.cuda.synchronize()
    return xs


def _eager(model, xs):
    outs, traces = {}, {}
    for M in MS:
        traces[M] = []
        outs[M] = model(xs[M], traces[M])
    torch.cuda.synchronize()
    return outs, traces


def test_model_graph_matches_oracle_per_layer(model):
    """One graph holds the three forwards (M = 1 on the lane-native copies, 8 and 32 on
    the pack() buffers: Layer_2_4.NATIVE_MAX_ROWS = 4; 384 GEMM calls); three replays
    equal the eager forward bit for bit, and every linear's output slice equals the
    oracle on its own input."""
    assert marlin.Layer_2_4.NATIVE_MAX_ROWS == 4 and MS == (1, 8, 32)
    xs = _inputs()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ref_out, _ = _eager(model, xs)  # also sizes the capture stream's split-K scratch
    for M in MS:
        assert torch.isfinite(ref_out[M]).all(), f"the synthetic stack overflowed at M={M}"
    g = torch.cuda.CUDAGraph()
    traces = {M: [] for M in MS}
    with torch.cuda.graph(g, stream=s):
        outs = {M: model(xs[M], traces[M]) for M in MS}
    for _ in range(3):
        for M in MS:
            outs[M].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for M in MS:
            assert torch.equal(outs[M], ref_out[M]), f"graph replay differs from eager at M={M}"
    for M in MS:
        assert len(traces[M]) == 4 * LAYERS
        for i, (name, inp, out) in enumerate(traces[M]):
            layer = getattr(model.layers[i // 4], name)
            chunks = layer.n // 64
            c0 = (7 * i + M) % (chunks - 1)
            t = _slice_packed(layer, c0, 2)
            ref = oracle_gemm(inp.cpu().numpy(), t)
            assert_close(out[:, 64 * c0:64 * (c0 + 2)].cpu().numpy(), ref, f"layer {i // 4} {name} M={M}")


def test_model_state_dict_round_trip(model):
    """state_dict -> bytes -> a fresh replace_linear'd model (weights_only load): the
    same outputs bit for bit, before and after to_native() on the fresh model."""
    sd = model.state_dict()
    assert all(k.rsplit(".", 1)[1] in ("B", "meta", "s") for k in sd), "only the pack() buffers persist"
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    fresh = _empty_model()
    fresh.load_state_dict(torch.load(buf, map_location=DEV, weights_only=True))
    xs = _inputs()
    ref_out, _ = _eager(model, xs)
    got32 = fresh(xs[32], [])
    torch.cuda.synchronize()
    assert torch.equal(got32, ref_out[32]), "M=32 (pack() buffers) differs after the round trip"
    _natives(fresh)
    got, _ = _eager(fresh, xs)
    for M in MS:
        assert torch.equal(got[M], ref_out[M]), f"M={M} differs after the round trip and to_native()"


def test_to_native_follows_load_state_dict():
    """A Layer_2_4 on the lane-native copy that then loads another weight's state_dict
    computes with the new weight at every batch size (the copy is rebuilt)."""
    K, N = 1024, 512
    layers = []
    for seed in (1, 2):
        wt = synth.make_weight(K, N, 600 + seed, 128, device=DEV)
        lay = marlin.Layer_2_4(K, N, groupsize=128).to(DEV)
        lay.B, lay.meta, lay.s = wt["B"], wt["meta"], wt["s"]
        layers.append(lay)
    first, second = layers
    first.to_native()
    first.load_state_dict(second.state_dict())
    t = {"B": second.B.cpu().numpy(), "meta": second.meta.cpu().numpy(), "s": second.s.cpu().numpy(), "K": K,
         "N": N, "groupsize": 128, "bits": 4}
    for M in (1, 16, 40):
        x = synth.make_activation(M, K, 610 + M, device=DEV)
        y = first(x)
        torch.cuda.synchronize()
        assert_close(y.cpu().numpy(), oracle_gemm(x.cpu().numpy(), t), f"after load_state_dict M={M}")
    # assign=True replaces the buffers themselves
    third = marlin.Layer_2_4(K, N, groupsize=128).to(DEV)
    wt = synth.make_weight(K, N, 603, 128, device=DEV)
    third.B, third.meta, third.s = wt["B"], wt["meta"], wt["s"]
    first.load_state_dict({k: v.clone() for k, v in third.state_dict().items()}, assign=True)
    t3 = {k: wt[k].cpu().numpy() for k in ("B", "meta", "s")}
    t3.update(K=K, N=N, groupsize=128, bits=4)
    x = synth.make_activation(4, K, 620, device=DEV)
    assert_close(first(x).cpu().numpy(), oracle_gemm(x.cpu().numpy(), t3), "after assign=True load")
