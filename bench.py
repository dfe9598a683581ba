"""Benchmark of the MI355X 2:4 INT4 x FP16 GEMM (libmarlin_hip.so).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode|decode70b|prefill|w3|meta3|stack]

Default workload (benchmark config "decode sweep"): Llama-2-7B projection shapes
(K x N = 4096x12288 QKV, 4096x4096 O, 4096x22016 gate/up, 11008x4096 down) at batch
M in {1, 2, 4, 8, 16}, 2:4 INT4 weights with group-128 fp16 scales.  One step is one
pass over the 20 (shape, M) calls, captured once in a HIP graph and replayed; the
weights rotate through copies totalling more than the 256 MB Infinity Cache so every
call streams its weight from HBM.  Prints ONE JSON line; ``value`` is the achieved
HBM bandwidth on algorithmic compressed-weight bytes (25/64*K*N per call).

Other workloads: ``decode70b`` (the decode sweep on the Llama-2-70B shapes below),
``native`` / ``native70b`` (the 7B / 70B decode shapes at M in {1, 2, 4, 8, 16} on the
lane-native layout of ``marlin.pack_native``), ``prefill`` (Llama-2-70B shapes, M in
{512..4096}, TFLOP/s),
``w3`` (3-bit values, M in {1, 16, 256}), ``meta3`` (3-bit metadata, decode sweep),
``dense`` (the decode sweep on the dense Marlin op ``marlin.mul``, GB/s on its K*N/2
code bytes plus scales), ``floor`` (per decode-sweep call: a plain streaming read of
its weight bytes and an empty kernel on its planned grid),
``stack`` (32 Llama-2-7B layers in sequence, M in {1, 8, 32}; ``stack_native`` runs
its M = 1 pass on the lane-native layout, as ``Layer_2_4.to_native()`` does), ``copy`` (a plain
1 GiB device copy: the calibration run for the HBM traffic counters), ``compare``
(per call site against hipBLASLt dense fp16 and hipSPARSELt 2:4 fp16).

``roofline.traffic`` is read from ``profiles/<workload>_hbm_traffic.md`` (HBM
bytes per launch from rocprofv3 FETCH_SIZE and WRITE_SIZE runs of this script,
scaled by the same counters on the ``copy`` workload); null when that file is
absent.  ``roofline.ceiling`` is the measured ceiling beside the published peak,
read from the committed profile of ``--workload floor`` / ``floor70b`` (a plain
streaming read of the same bytes) or ``mfma_floor`` (an MFMA-only stream of the
same smfmacs), with ``frac`` = achieved / ceiling.  ``--eager`` replays the calls without a graph (for counter runs).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import torch

from csed499ii_amd import _lib, marlin, synth

METRIC = "µs/call + achieved HBM GB/s (M=1–16) and TFLOP/s (M≥512), 2:4 INT4 GEMM"
HBM_PEAK_GBS = 8000.0
SPARSE_F16_PEAK_TFLOPS = 5000.0  # dense-equivalent FLOPs of 2:4 fp16 MFMA (2.5 PFLOP/s dense)
MALL_BYTES = 256 << 20

LLAMA7B = [("qkv", 4096, 12288), ("o", 4096, 4096), ("gate_up", 4096, 22016), ("down", 11008, 4096)]
LLAMA70B = [("qkv", 8192, 10240), ("o", 8192, 8192), ("gate_up", 8192, 57344), ("down", 28672, 8192)]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class WeightSet:
    """Copies of one packed weight, handed out round-robin to every call site that
    uses the shape, so that consecutive uses of one copy are separated by more
    bytes than the Infinity Cache holds."""

    def __init__(self, copies):
        self.copies = copies
        self.i = 0

    def next(self):
        w = self.copies[self.i % len(self.copies)]
        self.i += 1
        return w

    def reset(self):
        """Restart the round robin (before a capture, so that it counts its own uses)."""
        self.i = 0

    @property
    def used(self) -> int:
        """Distinct copies handed out since the last reset."""
        return min(self.i, len(self.copies))


class Call:
    """One GEMM call site."""

    def __init__(self, name, K, N, M, wset, A, fn, meta_key="meta"):
        self.name, self.K, self.N, self.M = name, K, N, M
        self.wset = wset
        self.A = A
        self.C = torch.empty((M, N), dtype=torch.half, device=A.device)
        self.ws = torch.zeros(N // 128 * 16, dtype=torch.int32, device=A.device)
        self.fn = fn
        self.meta_key = meta_key
        self.bits = wset.copies[0]["bits"]

    def __call__(self):
        w = self.wset.next()
        self.fn(self.A, w["B"], w[self.meta_key], self.C, w["s"], self.ws)

    @property
    def min_reps(self):
        """Calls per timing graph so that it cycles every copy of the weight (more
        than the Infinity Cache holds, when the copies were made for that)."""
        return len(self.wset.copies)

    @property
    def wbytes(self):
        if self.bits == "dense":
            return synth.dense_weight_bytes(self.K, self.N, 128)
        b = synth.weight_bytes(self.K, self.N, self.bits, 128)
        if self.meta_key == "meta3":
            b -= self.K * self.N // 8 // 4  # metadata is 3/4 of the 4-bit size
        return b

    @property
    def flops(self):
        return 2 * self.M * self.K * self.N

    @property
    def kb_bytes(self):
        """Bytes by the reference benchmark's formula (kernel_bench/bench.py:170):
        2 A.numel + 4 B.numel + 2 meta.numel + 2 C.numel + 2 s.numel, i.e. the
        weight bytes plus fp16 activations and outputs."""
        return self.wbytes + 2 * self.M * self.K + 2 * self.M * self.N


def kernel_of(c) -> str:
    """The kernel the library dispatches a call to: the lane-native kernel for the
    lane-native layout, the dense kernels for the dense op, else the first launch's
    kernel of the library's own plan (``marlin.plan_2_4``: the register-ring decode
    kernel at 1-8 padded rows, the LDS-DMA decode kernel at 16 and 32, the large-M
    kernel, or the general one)."""
    if getattr(c, "native", False):
        return "sm24::sm24_native_decode_kernel"
    if getattr(c, "bits", None) == "dense":
        big = c.M >= 65 and c.N % 512 == 0 and c.K % 128 == 0
        return "sm24::marlin_dense_prefill_kernel" if big else "sm24::marlin_dense_kernel"
    kind = marlin.plan_2_4(c.M, c.K, c.N, 128)["kernel"]
    return {"decode": "sm24::sm24_decode_kernel", "decode_dma": "sm24::sm24_decode_dma_kernel",
            "large_m": "sm24::sm24_prefill_kernel", "general": "sm24::sm24_gemm_kernel"}[kind]


def dense_fn(A, B, meta, C, s, ws):
    """Call-site adapter of the dense Marlin op (no metadata)."""
    marlin.mul(A, B, C, s, ws)


def make_copies(K, N, seed, bits, copies, device, meta3=False) -> WeightSet:
    if bits == "dense":
        base = synth.make_dense_weight(K, N, seed, 128, device=device)
    else:
        base = synth.make_weight(K, N, seed, 128, bits=bits, device=device)
    if meta3:
        base["meta3"] = marlin.pack_meta3(base["meta"].reshape(-1))
    out = [base]
    for _ in range(copies - 1):
        out.append({k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in base.items()})
    return WeightSet(out)


def copies_for(K, N, bits) -> int:
    """Copies of one weight whose total exceeds the Infinity Cache by 25 %."""
    wb = synth.dense_weight_bytes(K, N, 128) if bits == "dense" else synth.weight_bytes(K, N, bits, 128)
    return max(2, -(-int(MALL_BYTES * 1.25) // wb))


_STREAM = None


def capture_stream():
    """The stream every graph is warmed up and captured on: the library keeps its
    split-K scratch per stream, so the eager warm-up on this stream sizes the scratch
    that the captured calls then use."""
    global _STREAM
    if _STREAM is None:
        _STREAM = torch.cuda.Stream()
    return _STREAM


def graph_of(calls, reps=1):
    """Capture ``reps`` passes over ``calls`` into one graph, after an eager warm-up
    on the capture stream.  Each call site's weight round robin restarts at the
    capture, so ``WeightSet.used`` afterwards counts the copies the graph cycles."""
    s = capture_stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:
            c()
    torch.cuda.synchronize()
    for c in calls:
        if getattr(c, "wset", None) is not None:
            c.wset.reset()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(reps):
            for c in calls:
                c()
    torch.cuda.synchronize()
    return g


def time_graph(g, replays: int) -> float:
    """Median-free GPU time (ms) of ``replays`` back-to-back replays, HIP events on the
    stream the graph launches on."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        g.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end)


def per_call_stats(calls, samples=9, replays=5, reps=20, seed=20261019):
    """µs/call of every call site alone, by the reference's protocol
    (kernel_profile/run.py:80-99): a graph of at least ``reps`` calls per site, and
    enough to cycle all of its weight copies (weights rotating, so a replay streams
    more than the Infinity Cache holds), the (site, sample) jobs in a seeded random
    order, each sample one untimed replay then ``replays`` timed back-to-back
    replays; median over ``samples``."""
    import random

    graphs = [graph_of([c], reps=max(reps, getattr(c, "min_reps", 1))) for c in calls]
    nreps = [max(reps, getattr(c, "min_reps", 1)) for c in calls]
    jobs = [(i, k) for i in range(len(calls)) for k in range(samples)]
    random.Random(seed).shuffle(jobs)
    ts = [[] for _ in calls]
    for i, _ in jobs:
        graphs[i].replay()
        ts[i].append(time_graph(graphs[i], replays) * 1000.0 / (replays * nreps[i]))
    out = []
    for c, t in zip(calls, ts):
        us = statistics.median(t)
        row = {"name": c.name, "M": c.M, "K": c.K, "N": c.N, "us": round(us, 3),
               "GBps": round(c.wbytes / (us * 1e3), 1), "kb_bench_GBps": round(c.kb_bytes / (us * 1e3), 1)}
        if c.M >= 256:
            row["TFLOPs"] = round(c.flops / (us * 1e6), 1)
        out.append(row)
    del graphs
    return out


def cpu_threads() -> int:
    """Host threads the CPU baseline runs on: the CPUs this process may use, capped by
    OMP_NUM_THREADS when that is set (the GPU boxes give one GPU's job a share of
    the host's cores)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(decode_shapes=LLAMA7B, decode_ms=(1, 16), prefill=(("o", 8192, 8192), 512), reps=3):
    """The reference's CPU path on the host cores: the packed
    weight is unpacked and dequantized once by the oracle (timed separately: a
    one-time cost), then each call is ``torch.matmul(A.float(), W.float())`` in fp32
    with ``torch.set_num_threads`` = the host threads available; one warm-up and
    ``reps`` timed calls, median.  ``value`` is GB/s of algorithmic compressed-weight
    bytes over the decode calls (the four Llama-2-7B shapes at M in {1, 16}), the
    same bytes as the GPU line; the Llama-2-70B O projection at M = 512 is reported
    in TFLOP/s beside it."""
    import numpy as np

    from oracle import sm24_oracle as o

    threads = cpu_threads()
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        calls, dequant_s = [], {}
        shapes = [(n, K, N, decode_ms) for n, K, N in decode_shapes] + [(prefill[0][0] + "_70b", prefill[0][1],
                                                                          prefill[0][2], (prefill[1],))]
        for i, (name, K, N, Ms) in enumerate(shapes):
            wt = synth.make_weight(K, N, synth.SEED_BASE + 1 + i, 128, device="cpu")
            t0 = time.perf_counter()
            W = torch.from_numpy(o.dequant(wt["B"].numpy(), wt["meta"].numpy(), wt["s"].numpy(), K, N, 128))
            dequant_s[name] = time.perf_counter() - t0
            W32 = W.float()
            del wt, W
            for M in Ms:
                A = synth.make_activation(M, K, synth.SEED_BASE + M, device="cpu")
                torch.matmul(A.float(), W32)  # warm-up
                ts = []
                for _ in range(reps):
                    t0 = time.perf_counter()
                    torch.matmul(A.float(), W32)
                    ts.append(time.perf_counter() - t0)
                calls.append({"name": name, "M": M, "K": K, "N": N, "us": statistics.median(ts) * 1e6})
            del W32
    finally:
        torch.set_num_threads(prev_threads)
    dec = [c for c in calls if c["M"] <= 16]
    wbytes = sum(synth.weight_bytes(c["K"], c["N"], 4, 128) for c in dec)
    dec_us = sum(c["us"] for c in dec)
    pre = [c for c in calls if c["M"] > 16]
    for c in calls:
        c["us"] = round(c["us"], 1)
        c["GBps"] = round(synth.weight_bytes(c["K"], c["N"], 4, 128) / (c["us"] * 1e3), 3)
        c["TFLOPs"] = round(2 * c["M"] * c["K"] * c["N"] / (c["us"] * 1e6), 4)
    sample = (f"reference CPU path restated: oracle dequantize once per weight (timed apart: "
              + ", ".join(f"{k} {v:.2f} s" for k, v in dequant_s.items())
              + f"), then fp32 torch.matmul per call on {threads} threads, median of {reps} after 1 warm-up; "
              f"value over the 8 decode calls (Llama-2-7B qkv/o/gate_up/down at M in {{1, 16}}); "
              f"Llama-2-70B o at M=512 in prefill_TFLOPs")
    return {"value": round(wbytes / (dec_us * 1e3), 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": sample, "host_cpu_count": os.cpu_count(), "calls": calls,
            "dequant_s": {k: round(v, 3) for k, v in dequant_s.items()},
            "prefill_TFLOPs": pre[0]["TFLOPs"] if pre else None}


class LibCall:
    """Dense fp16 ``torch.matmul`` (hipBLASLt) at one call site, for the ``compare``
    workload, on random 2:4-pruned fp16 weights of the same shape (values do not
    matter for timing), rotating through copies like ``Call``."""

    def __init__(self, name, K, N, M, kind, A, copies):
        self.name, self.K, self.N, self.M, self.kind = name, K, N, M, kind
        self.A = A
        self.ws = []
        for c in range(copies):
            w = (torch.randn((K, N), device=A.device) * 0.02).to(torch.float16)
            w = w * synth.prune_2_4(w)
            self.ws.append(w)
        self.i = 0

    def __call__(self):
        w = self.ws[self.i % len(self.ws)]
        self.i += 1
        return torch.matmul(self.A, w)


class SparseLtCall:
    """hipSPARSELt 2:4 fp16 GEMM at one call site (``libhipsparselt`` through ctypes,
    default algorithm, fp32 compute): D[N, Mp] = W^T[N, K] (pruned and compressed by
    the library) x X^T[K, Mp] with Mp = max(M, 16); random weights of the shape, the
    compressed copies rotating like ``Call``."""

    _lib = None
    _handle = None

    @classmethod
    def lib(cls):
        if cls._lib is None:
            import ctypes
            for name in ("libhipsparselt.so", "/opt/rocm/lib/libhipsparselt.so"):
                try:
                    cls._lib = ctypes.CDLL(name)
                    break
                except OSError:
                    continue
            if cls._lib is None:
                raise RuntimeError("libhipsparselt.so not found")
            cls._handle = ctypes.create_string_buffer(11024)
            cls._check("hipsparseLtInit", cls._lib.hipsparseLtInit(cls._handle))
        return cls._lib

    @staticmethod
    def _check(fn, status):
        if status != 0:
            raise RuntimeError(f"{fn} returned status {status}")

    def __init__(self, name, K, N, M, copies, device):
        import ctypes
        lib = self.lib()
        h = self._handle
        c_i64, vp = ctypes.c_int64, ctypes.c_void_p
        self.name, self.K, self.N, self.M = name, K, N, M
        Mp = max(M, 16)
        f16, row, nt, f32c, alg, strip = 2, 2, 0, 2, 0, 1
        self.desc = [ctypes.create_string_buffer(11024) for _ in range(3)]
        self.md, self.alg, self.plan = (ctypes.create_string_buffer(11024) for _ in range(3))
        chk = self._check
        chk("StructuredDescriptorInit", lib.hipsparseLtStructuredDescriptorInit(
            h, self.desc[0], c_i64(N), c_i64(K), c_i64(K), ctypes.c_uint32(16), f16, row, 0))
        chk("DenseDescriptorInit", lib.hipsparseLtDenseDescriptorInit(
            h, self.desc[1], c_i64(K), c_i64(Mp), c_i64(Mp), ctypes.c_uint32(16), f16, row))
        chk("DenseDescriptorInit", lib.hipsparseLtDenseDescriptorInit(
            h, self.desc[2], c_i64(N), c_i64(Mp), c_i64(Mp), ctypes.c_uint32(16), f16, row))
        chk("MatmulDescriptorInit", lib.hipsparseLtMatmulDescriptorInit(
            h, self.md, nt, nt, self.desc[0], self.desc[1], self.desc[2], self.desc[2], f32c))
        chk("MatmulAlgSelectionInit", lib.hipsparseLtMatmulAlgSelectionInit(h, self.alg, self.md, alg))
        chk("MatmulPlanInit", lib.hipsparseLtMatmulPlanInit(h, self.plan, self.md, self.alg))
        ws, csize, cbuf = ctypes.c_size_t(0), ctypes.c_size_t(0), ctypes.c_size_t(0)
        chk("MatmulGetWorkspace", lib.hipsparseLtMatmulGetWorkspace(h, self.plan, ctypes.byref(ws)))
        chk("SpMMACompressedSize", lib.hipsparseLtSpMMACompressedSize(h, self.plan, ctypes.byref(csize),
                                                                      ctypes.byref(cbuf)))
        self.B = torch.randn((K, Mp), device=device).to(torch.float16)
        self.D = torch.empty((N, Mp), dtype=torch.float16, device=device)
        self.ws = torch.empty(max(ws.value, 1), dtype=torch.uint8, device=device)
        cb = torch.empty(max(cbuf.value, 1), dtype=torch.uint8, device=device)
        stream = vp(torch.cuda.current_stream().cuda_stream)
        self.comp = []
        for _ in range(copies):
            w = (torch.randn((N, K), device=device) * 0.02).to(torch.float16)
            chk("SpMMAPrune", lib.hipsparseLtSpMMAPrune(h, self.md, vp(w.data_ptr()), vp(w.data_ptr()), strip,
                                                         stream))
            c = torch.empty(csize.value, dtype=torch.uint8, device=device)
            chk("SpMMACompress", lib.hipsparseLtSpMMACompress(h, self.plan, vp(w.data_ptr()), vp(c.data_ptr()),
                                                               vp(cb.data_ptr()), stream))
            self.comp.append(c)
        torch.cuda.synchronize()
        self.alpha, self.beta = ctypes.c_float(1.0), ctypes.c_float(0.0)
        self.i = 0

    def __call__(self):
        import ctypes
        vp = ctypes.c_void_p
        c = self.comp[self.i % len(self.comp)]
        self.i += 1
        stream = vp(torch.cuda.current_stream().cuda_stream)
        self._check("Matmul", self.lib().hipsparseLtMatmul(
            self._handle, self.plan, ctypes.byref(self.alpha), vp(c.data_ptr()), vp(self.B.data_ptr()),
            ctypes.byref(self.beta), vp(self.D.data_ptr()), vp(self.D.data_ptr()), vp(self.ws.data_ptr()),
            ctypes.byref(stream), 1))


def time_site(fn, reps=20, samples=5):
    """µs per call of ``fn``: a captured graph of ``reps`` calls, or (when the library
    call cannot be captured) ``reps`` eager calls between two events; median of
    ``samples``.  The warm-up call runs on the capture stream, so that a call that
    splits K has that stream's scratch when it is captured.  Returns (µs, method)."""
    s = capture_stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(reps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        run, method = g.replay, "graph"
    except Exception:  # noqa: BLE001 - library not capturable: time it eagerly
        torch.cuda.synchronize()

        def run():
            for _ in range(reps):
                fn()
        method = "eager"
    ts = []
    for _ in range(samples):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1000.0 / reps)
    return statistics.median(ts), method


def compare_libraries(device):
    """Per call site: this library's mul_2_4 against hipBLASLt dense fp16 and
    hipSPARSELt 2:4 fp16 (M padded to 16) at the decode (Llama-2-7B, M in {1, 16})
    and prefill (Llama-2-70B, M in {512, 2048}) shapes."""
    rows = []
    cases = [(n, K, N, M) for M in (1, 16) for (n, K, N) in LLAMA7B] + \
            [(n, K, N, M) for M in (512, 2048) for (n, K, N) in LLAMA70B]
    for i, (name, K, N, M) in enumerate(cases):
        decode = M <= 32
        A = synth.make_activation(M, K, synth.SEED_BASE + M, device=device)
        log(f"bench: compare {name} M={M}")
        ours = Call(name, K, N, M, make_copies(K, N, synth.SEED_BASE + 1 + i, 4,
                                               copies_for(K, N, 4) if decode else 1, device), A, marlin.mul_2_4)
        row = {"name": name, "M": M, "K": K, "N": N}
        row["ours_us"], _ = time_site(ours)
        if M <= 16:  # the same weights repacked to the lane-native layout
            nat_copies = []
            for w in ours.wset.copies:
                Bn, Mn, Sn = marlin.pack_native(w["B"], w["meta"], w["s"])
                nat_copies.append({"B": Bn, "meta": Mn, "s": Sn, "bits": 4})

            def native_fn(A_, B, meta, C, s, ws):
                marlin.mul_2_4_native(A_, B, meta, C, s)
            row["ours_native_us"], _ = time_site(Call(name, K, N, M, WeightSet(nat_copies), A, native_fn))
            del nat_copies
        del ours
        # the sibling op: this library's dense Marlin INT4 x FP16 GEMM (marlin.mul)
        dense = Call(name, K, N, M, make_copies(K, N, synth.SEED_BASE + 51 + i, "dense",
                                                copies_for(K, N, "dense") if decode else 1, device), A, dense_fn)
        row["ours_dense_marlin_us"], _ = time_site(dense)
        del dense
        for kind, key in (("dense", "dense_fp16_hipblaslt_us"), ("sparse", "sparse24_fp16_hipsparselt_us")):
            fp16_bytes = 2 * K * N // (1 if kind == "dense" else 2)
            copies = max(2, -(-int(MALL_BYTES * 1.25) // fp16_bytes)) if decode else 1
            try:
                site = LibCall(name, K, N, M, kind, A, copies) if kind == "dense" else \
                    SparseLtCall(name, K, N, M, copies, device)
                row[key], row[key.replace("_us", "_timing")] = time_site(site)
                del site
            except Exception as e:  # noqa: BLE001 - report a library that does not run here
                row[key] = None
                row[key.replace("_us", "_error")] = f"{type(e).__name__}: {str(e)[:160]}"
            torch.cuda.empty_cache()
        for key in ("ours_us", "ours_native_us", "ours_dense_marlin_us", "dense_fp16_hipblaslt_us",
                    "sparse24_fp16_hipsparselt_us"):
            if row.get(key) is not None:
                row[key] = round(row[key], 2)
        rows.append(row)
    return rows


def build_workload(args, device):
    wl = args.workload
    calls = []
    if wl in ("decode", "decode70b", "meta3", "w3", "dense"):
        shapes = LLAMA70B if wl == "decode70b" else LLAMA7B
        Ms = [1, 2, 4, 8, 16] if wl != "w3" else [1, 16, 256]
        bits = 3 if wl == "w3" else ("dense" if wl == "dense" else 4)
        weights = {}
        copies = {}
        for i, (name, K, N) in enumerate(shapes):
            copies[name] = copies_for(K, N, bits)
            weights[name] = make_copies(K, N, synth.SEED_BASE + 1 + i, bits, copies[name], device,
                                        meta3=(wl == "meta3"))
        fn = {"w3": marlin.mul_2_4_w3, "meta3": marlin.mul_2_4_meta3, "dense": dense_fn}.get(wl, marlin.mul_2_4)
        meta_key = "meta3" if wl == "meta3" else "meta"
        for M in Ms:
            for name, K, N in shapes:
                A = synth.make_activation(M, K, synth.SEED_BASE + M, device=device)
                calls.append(Call(name, K, N, M, weights[name], A, fn, meta_key))
        cfg = {"workload": {"decode": "decode_sweep_llama2_7b", "decode70b": "decode_sweep_llama2_70b",
                            "meta3": "decode_sweep_llama2_7b_meta3", "w3": "w3_values_llama2_7b",
                            "dense": "dense_marlin_decode_sweep_llama2_7b"}[wl],
               "M": Ms, "shapes_KxN": [f"{K}x{N}" for _, K, N in shapes], "groupsize": 128,
               "weight_copies_made": copies}
    elif wl in ("native", "native70b"):
        shapes = LLAMA70B if wl == "native70b" else LLAMA7B
        Ms = [1, 2, 4, 8, 16]
        weights, copies = {}, {}
        for i, (name, K, N) in enumerate(shapes):
            copies[name] = copies_for(K, N, 4)
            base = synth.make_weight(K, N, synth.SEED_BASE + 1 + i, 128, device=device)
            Bn, Mn, Sn = marlin.pack_native(base["B"], base["meta"], base["s"])
            nat = {"B": Bn, "meta": Mn, "s": Sn, "bits": 4}
            weights[name] = WeightSet([nat] + [{k: (v.clone() if isinstance(v, torch.Tensor) else v)
                                                for k, v in nat.items()} for _ in range(copies[name] - 1)])

        def native_fn(A, B, meta, C, s, ws):
            marlin.mul_2_4_native(A, B, meta, C, s)
        for M in Ms:
            for name, K, N in shapes:
                A = synth.make_activation(M, K, synth.SEED_BASE + M, device=device)
                calls.append(Call(name, K, N, M, weights[name], A, native_fn))
                calls[-1].native = True
        cfg = {"workload": "native_decode_llama2_70b" if wl == "native70b" else "native_decode_llama2_7b",
               "M": Ms, "shapes_KxN": [f"{K}x{N}" for _, K, N in shapes], "groupsize": 128, "layout": "lane-native",
               "weight_copies_made": copies}
    elif wl == "prefill":
        Ms = args.prefill_m
        for i, (name, K, N) in enumerate(LLAMA70B):
            w = make_copies(K, N, synth.SEED_BASE + 11 + i, 4, 1, device)
            for M in Ms:
                A = synth.make_activation(M, K, synth.SEED_BASE + M, device=device)
                calls.append(Call(name, K, N, M, w, A, marlin.mul_2_4))
        cfg = {"workload": "prefill_sweep_llama2_70b", "M": Ms, "shapes_KxN": [f"{K}x{N}" for _, K, N in LLAMA70B],
               "groupsize": 128}
    elif wl in ("stack", "stack_native"):
        Ms = [1, 8, 32]
        native = wl == "stack_native"
        layers, nlayers = [], []
        for l in range(32):
            layers.append({name: make_copies(K, N, synth.SEED_BASE + 1000 + 4 * l + i, 4, 1, device)
                           for i, (name, K, N) in enumerate(LLAMA7B)})
            if native:
                nl = {}
                for name, ws in layers[-1].items():
                    w = ws.copies[0]
                    Bn, Mn, Sn = marlin.pack_native(w["B"], w["meta"], w["s"])
                    nl[name] = WeightSet([{"B": Bn, "meta": Mn, "s": Sn, "bits": 4}])
                nlayers.append(nl)

        def native_fn(A, B, meta, C, s, ws):
            marlin.mul_2_4_native(A, B, meta, C, s)
        for M in Ms:
            As = {K: synth.make_activation(M, K, synth.SEED_BASE + M, device=device) for _, K, _ in LLAMA7B}
            for l in range(32):
                for name, K, N in LLAMA7B:
                    if native and M <= marlin.Layer_2_4.NATIVE_MAX_ROWS:  # what Layer_2_4.to_native() runs
                        calls.append(Call(f"L{l}.{name}", K, N, M, nlayers[l][name], As[K], native_fn))
                        calls[-1].native = True
                    else:
                        calls.append(Call(f"L{l}.{name}", K, N, M, layers[l][name], As[K], marlin.mul_2_4))
        cfg = {"workload": "decode_stack_32x_llama2_7b" + ("_native" if native else ""), "M": Ms, "layers": 32,
               "groupsize": 128}
        if native:
            cfg["layout"] = (f"lane-native for M <= {marlin.Layer_2_4.NATIVE_MAX_ROWS} (Layer_2_4.to_native), "
                             "pack() layout above")
    elif wl == "copy":
        n = (1 << 30) // 2
        src = torch.ones(n, dtype=torch.half, device=device)
        dst = torch.empty_like(src)

        class Copy:
            name, K, N, M = "copy", 0, 0, 0
            wbytes = 2 * n  # bytes read (and as many written)
            kb_bytes = 4 * n  # read + written
            flops = 0

            def __call__(self):
                dst.copy_(src)

        calls = [Copy()]
        cfg = {"workload": "copy_1gib", "bytes_read": 2 * n, "bytes_written": 2 * n}
    else:
        raise SystemExit(f"unknown workload {wl}")
    return calls, cfg


def traffic_from_profile(workload: str):
    """HBM bytes per launch recorded in profiles/<workload>_hbm_traffic.md (a line
    ``traffic_bytes_per_launch: <int>``), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{workload}_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        return None
    return None


# Measured ceilings beside the published peaks: the profile that records each, the
# line holding the figure, and the regular expression of the figure in it.
CEILINGS = {
    "decode_sweep_llama2_7b": ("decode_floor_llama2_7b.md", "Sum over the 20 calls", r"\(([0-9.]+) GB/s", "GB/s",
                               "plain streaming read of each call's weight bytes, summed over the sweep "
                               "(bench.py --workload floor)"),
    "decode_sweep_llama2_70b": ("decode_floor_llama2_70b.md", "Sum over the 20 calls", r"\(([0-9.]+) GB/s", "GB/s",
                                "plain streaming read of each call's weight bytes, summed over the sweep "
                                "(bench.py --workload floor70b)"),
    "prefill_sweep_llama2_70b": ("prefill_mfma_floor.md", "Sweep: the MFMA-only stream", r"\(([0-9.]+) TFLOP/s",
                                 "TFLOP/s", "MFMA-only smfmac stream on each call's planned grid with its smfmac "
                                            "count, summed over the sweep (bench.py --workload mfma_floor)"),
}


def ceiling_from_profile(workload: str, achieved: float):
    """The measured ceiling of ``workload`` from its committed profile, as
    {value, unit, frac (achieved / value), source, what}, or None."""
    import re

    if workload not in CEILINGS:
        return None
    fname, key, pat, unit, what = CEILINGS[workload]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", fname)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key):
                    m = re.search(pat, line)
                    if m:
                        v = float(m.group(1))
                        return {"value": v, "unit": unit, "frac": round(achieved / v, 4), "source": f"profiles/{fname}",
                                "what": what}
    except OSError:
        return None
    return None


class ProbeRead:
    """The floor workload's stand-in for one decode call: a plain streaming read of the
    call's algorithmic weight bytes (libmarlin_probe.so), each call reading the next
    window of a pool larger than the Infinity Cache."""

    lib = None

    def __init__(self, c, pool, sink, blocks):
        self.name, self.K, self.N, self.M = c.name, c.K, c.N, c.M
        self.wbytes = c.wbytes
        self.kb_bytes = c.kb_bytes
        self.flops = c.flops
        self.nbytes = -(-c.wbytes // 4096) * 4096
        self.pool, self.sink, self.blocks = pool, sink, blocks
        self.off = 0
        self.wset = None
        self.min_reps = -(-int(MALL_BYTES * 1.25) // self.nbytes)

    def __call__(self):
        span = self.pool.numel() - self.nbytes
        self.off = (self.off + self.nbytes + 65536) % span
        p = self.pool.data_ptr() + self.off // 4096 * 4096
        err = self.lib.marlin_probe_read(ctypes.c_void_p(p), self.nbytes, ctypes.c_void_p(self.sink.data_ptr()),
                                         self.blocks, self.pool.get_device(),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if err:
            raise RuntimeError(f"marlin_probe_read error {err}")


class ProbeEmpty:
    """An empty kernel on the grid the library plans for one decode call."""

    lib = None

    def __init__(self, c, device):
        self.name, self.K, self.N, self.M = c.name, c.K, c.N, c.M
        self.wbytes, self.kb_bytes, self.flops = 0, 0, 0
        self.plan = marlin.plan_2_4(c.M, c.K, c.N, 128)
        self.dev = torch.device(device).index or 0
        self.wset = None

    def __call__(self):
        err = self.lib.marlin_probe_empty(self.plan["workgroups"], self.plan["threads"], self.dev,
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if err:
            raise RuntimeError(f"marlin_probe_empty error {err}")


def load_probe():
    from csed499ii_amd import build as _build

    if ProbeRead.lib is None:
        if not _build.PROBE_LIB.exists():
            raise RuntimeError(f"{_build.PROBE_LIB.name} is not built; run `python -m csed499ii_amd.build`")
        lib = ctypes.CDLL(str(_build.PROBE_LIB))
        lib.marlin_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_void_p]
        lib.marlin_probe_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        lib.marlin_probe_smfmac_stream.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                                   ctypes.c_int, ctypes.c_void_p]
        ProbeRead.lib = ProbeEmpty.lib = SmfmacStream.lib = lib
    return ProbeRead.lib


class SmfmacStream:
    """The mfma_floor workload's stand-in for one prefill call: the MFMA-only stream of
    libmarlin_probe.so on the call's planned grid (workgroups of 8 waves, 128
    accumulator AGPRs each), with as many v_smfmac_f32_32x32x32_f16 per SIMD as the
    call issues per 64-deep k-step: 32 (two waves of 16) for 512x128 tiles, 16 for
    64-row tiles (two waves of 8) and for the narrow 256x128 tiles (one wave of 16)."""

    lib = None

    def __init__(self, c, device):
        self.name, self.K, self.N, self.M = c.name, c.K, c.N, c.M
        self.wbytes, self.kb_bytes, self.flops = 0, 0, c.flops
        self.plan = marlin.plan_2_4(c.M, c.K, c.N, 128)
        tiles = self.plan["workgroups"] // self.plan["splits"]
        self.narrow = self.plan["threads"] == 256
        self.rows = 128 if self.narrow or tiles == (c.N // 512) * -(-c.M // 128) else 64
        ksteps = -(-(c.K // 64) // self.plan["splits"])
        self.iters = max(1, ksteps // 2 if self.narrow else ksteps * self.rows // 128)
        self.dev = torch.device(device).index or 0
        self.out = torch.zeros(self.plan["workgroups"] * 8, dtype=torch.float32, device=device)
        self.clock = torch.zeros(4, dtype=torch.int64, device=device)
        self.wset = None

    def __call__(self):
        err = self.lib.marlin_probe_smfmac_stream(self.plan["workgroups"], self.iters,
                                                  ctypes.c_void_p(self.out.data_ptr()),
                                                  ctypes.c_void_p(self.clock.data_ptr()), self.dev,
                                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if err:
            raise RuntimeError(f"marlin_probe_smfmac_stream error {err}")


def mfma_floor_workload(args, device, cus=256):
    """The compute ceiling of the prefill sweep: per call, the MFMA-only smfmac stream
    on the call's grid (SmfmacStream) beside the call itself, both by the reference
    protocol.  The stream's clock is its wave 0's shader clock against the real-time
    counter (one sample per call); cycles per smfmac = clock x time / (rounds of
    workgroups over the CUs x smfmacs per SIMD: 2 waves x 16 per iteration)."""
    load_probe()
    sub = argparse.Namespace(**vars(args))
    sub.workload = "prefill"
    calls, _ = build_workload(sub, device)
    rows = []
    for c in calls:
        st = SmfmacStream(c, device)
        su = per_call_stats([st], samples=5, replays=2, reps=4)[0]["us"]
        cl = st.clock.cpu().tolist()
        ghz = (cl[2] - cl[0]) / max(cl[3] - cl[1], 1) * 0.1  # 100 MHz real-time ticks
        gu = per_call_stats([c], samples=5, replays=2, reps=4)[0]["us"]
        rounds = -(-st.plan["workgroups"] // cus)
        smf = rounds * st.iters * 32
        rows.append({"name": c.name, "M": c.M, "K": c.K, "N": c.N, "tile_rows": st.rows,
                     "tile_cols": 256 if st.narrow else 512,
                     "splits": st.plan["splits"], "workgroups": st.plan["workgroups"],
                     "stream_us": su, "stream_TFLOPs": round(c.flops / (su * 1e6), 1),
                     "stream_clock_GHz": round(ghz, 2),
                     "stream_cycles_per_smfmac": round(ghz * 1e3 * su / smf, 1),
                     "gemm_us": gu, "gemm_TFLOPs": round(c.flops / (gu * 1e6), 1),
                     "gemm_of_stream": round(su / gu, 3)})
        log(f"bench: mfma floor {c.name} M={c.M}: stream {su:.1f} us ({rows[-1]['stream_TFLOPs']} TFLOP/s, "
            f"{ghz:.2f} GHz, {rows[-1]['stream_cycles_per_smfmac']} cycles/smfmac), gemm {gu:.1f} us")
    return rows


def floor_workload(args, device, shapes_70b=False):
    """The per-call floor of the decode sweep (Llama-2-7B shapes, or -70B with
    ``shapes_70b``): for every (shape, M) call, a streaming read of exactly its weight
    bytes (best of several grid sizes) and an empty kernel on its planned grid, each
    timed by the reference protocol.  The floor of a call is the read (a kernel that
    moves those bytes cannot take less); the empty kernel is its launch share."""
    load_probe()
    sub = argparse.Namespace(**vars(args))
    sub.workload = "decode70b" if shapes_70b else "decode"
    calls, _ = build_workload(sub, device)
    pool = torch.empty(int(MALL_BYTES * 1.5) + (64 << 20), dtype=torch.uint8, device=device)
    pool.random_(0, 256)
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    rows = []
    for c in calls:
        best = None
        for blocks in (256, 512, 1024, 2048, -256, -512, -1024, -2048):  # < 0: a contiguous range per wave
            r = per_call_stats([ProbeRead(c, pool, sink, blocks)])[0]
            if best is None or r["us"] < best[0]:
                best = (r["us"], blocks)
        e = ProbeEmpty(c, device)
        eu = per_call_stats([e])[0]["us"]
        rows.append({"name": c.name, "M": c.M, "K": c.K, "N": c.N, "read_us": best[0], "read_blocks": best[1],
                     "read_GBps": round(c.wbytes / (best[0] * 1e3), 1), "empty_us": eu,
                     "workgroups": e.plan["workgroups"], "threads": e.plan["threads"]})
        log(f"bench: floor {c.name} M={c.M}: read {best[0]:.2f} us ({abs(best[1])} blocks, "
            f"{'per-wave ranges' if best[1] < 0 else 'grid stride'}), empty {eu:.2f} us")
    del pool
    return rows


def span_row(c, plan, t):
    """Summary of one launch's per-wave stamps ``t`` [waves, 12] (see spans_workload)."""
    import numpy as np

    t0, targ, tset, t1, t2, t3, c0, c1 = (t[:, i] for i in range(8))
    if (t0 == 0).any():
        raise RuntimeError(f"spans: {c.name} M={c.M}: some waves recorded nothing")

    def med(x):
        return round(float(np.median(x)) / 100.0, 3)  # 100 MHz ticks -> us

    def mx(x):
        return round(float(np.max(x)) / 100.0, 3)

    clk = float(np.median((c1 - c0) / np.maximum(t3 - t0, 1))) * 100.0 / 1000.0  # GHz

    # the waves that end the call: the latest-ending 1 %, their phases on average
    end = t3 - t0.min()
    crit = end >= np.percentile(end, 99)

    def cm(x):
        return round(float(np.mean(x[crit])) / 100.0, 3)

    # waves per compute unit (word 8: the wave's XCC, shader engine and CU id) and the
    # median main loop of the waves on CUs of each load
    cu_ids, cu_inv, cu_waves = np.unique(t[:, 8], return_inverse=True, return_counts=True)
    load = cu_waves[cu_inv]
    by_load = {int(v): {"cus": int((cu_waves == v).sum()), "loop_us": med((t2 - t1)[load == v])}
               for v in np.unique(cu_waves)}
    return {"name": c.name, "M": c.M, "K": c.K, "N": c.N, "workgroups": plan["workgroups"],
            "waves": plan["threads"] // 64,
            "span_us": mx(t3 - t0.min()), "start_spread_us": mx(t0 - t0.min()),
            "args_us": med(targ - t0), "setup_us": med(tset - targ), "issue_us": med(t1 - tset),
            "prologue_us": med(t1 - t0), "prologue_max_us": mx(t1 - t0),
            "loop_us": med(t2 - t1), "loop_max_us": mx(t2 - t1),
            "tail_us": med(t3 - t2), "tail_max_us": mx(t3 - t2),
            "wave_us": med(t3 - t0), "clock_GHz": round(clk, 2),
            "last_waves": {"start_us": cm(t0 - t0.min()), "prologue_us": cm(t1 - t0), "loop_us": cm(t2 - t1),
                           "tail_us": cm(t3 - t2)},
            "cus": len(cu_ids), "waves_per_cu": by_load,
            "first_start": int(t0.min()), "last_end": int(t3.max())}


def spans_in_sweep(calls, set_spans, device):
    """Stamps of every call of one pass of the bench's decode graph (the default
    workload's step: the calls back to back, weights rotating), each call with its
    own buffer; the last of 5 replays.  Adds the gap from the previous call's last
    wave exit to this call's first wave entry."""
    plans = [marlin.plan_2_4(c.M, c.K, c.N, 128) for c in calls]
    bufs = [torch.zeros(p["workgroups"] * (p["threads"] // 64) * 12, dtype=torch.int64, device=device)
            for p in plans]
    s = capture_stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:
            c()
    torch.cuda.synchronize()
    for c in calls:
        c.wset.reset()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        try:
            for c, b in zip(calls, bufs):
                set_spans(ctypes.c_void_p(b.data_ptr()))
                c()
        finally:
            set_spans(None)
    for _ in range(5):
        g.replay()
    torch.cuda.synchronize()
    rows, prev_end = [], None
    for c, p, b in zip(calls, plans, bufs):
        r = span_row(c, p, b.view(-1, 12).cpu().numpy().astype("int64"))
        r["gap_us"] = None if prev_end is None else round((r["first_start"] - prev_end) / 100.0, 3)
        prev_end = r["last_end"]
        rows.append(r)
        log(f"bench: sweep spans {c.name} M={c.M}: gap {r['gap_us']} us, span {r['span_us']} us, "
            f"start spread {r['start_spread_us']}, prologue {r['prologue_us']} (args {r['args_us']}, "
            f"setup {r['setup_us']}, issue {r['issue_us']}), loop {r['loop_us']} (max {r['loop_max_us']}), "
            f"tail {r['tail_us']} (max {r['tail_max_us']})")
    del g
    return rows


def spans_workload(args, device, shapes_70b=False, in_sweep=False):
    """Per-wave phase timestamps of every decode-sweep call (the measurement build
    ``libmarlin_hip_spans.so``, whose decode kernel records the 100 MHz real-time
    counter at entry, once its first stages' loads are issued, after its last stage
    and at exit).  Each call site is captured in a graph of 40 back-to-back calls
    (weights rotating through their copies) whose last two calls carry stamp buffers,
    replayed 5 times; the last replay's stamps are summarised: the gap from the
    previous call's last wave exit to this call's first wave entry, the span from the
    first wave's entry to the last wave's exit, the spread of wave entries, and per
    wave the
    median and maximum of the prologue (entry to first loads issued; its median
    split into the wait for the kernel arguments, the load-address setup and the
    issue of the first stages' loads), the main loop (to the last stage's MFMAs) and
    the reduction and store (to exit); the same phases averaged over the waves that
    end the call (the latest-ending 1 %); and how many waves each compute unit ran,
    with the median main loop at each load.  ``in_sweep``: the same for every call
    of one pass of the default workload's graph (spans_in_sweep)."""
    from csed499ii_amd import build as _build

    lib = _lib.load()
    set_spans = lib.marlin_hip_set_spans
    set_spans.restype = ctypes.c_int
    set_spans.argtypes = [ctypes.c_void_p]
    if set_spans(None) != 0:
        raise SystemExit(f"{_lib.LIB_PATH.name} records no stamps: the spans workload needs {_build.SPANS_LIB.name}")
    sub = argparse.Namespace(**vars(args))
    sub.workload = "decode70b" if shapes_70b else "decode"
    calls, _ = build_workload(sub, device)
    if in_sweep:
        return spans_in_sweep(calls, set_spans, device)
    rows = []
    for c in calls:
        plan = marlin.plan_2_4(c.M, c.K, c.N, 128)
        waves = plan["threads"] // 64
        nwaves = plan["workgroups"] * waves
        prev = torch.zeros(nwaves * 12, dtype=torch.int64, device=device)
        buf = torch.zeros(nwaves * 12, dtype=torch.int64, device=device)
        s = capture_stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            c()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(38):
                c()
            try:
                for b in (prev, buf):
                    set_spans(ctypes.c_void_p(b.data_ptr()))
                    c()
            finally:
                set_spans(None)
        for _ in range(5):
            g.replay()
        torch.cuda.synchronize()
        t = buf.view(nwaves, 12).cpu().numpy().astype("int64")
        prev_end = int(prev.view(nwaves, 12)[:, 5].max())
        del g
        row = span_row(c, plan, t)
        row["gap_us"] = round((row["first_start"] - prev_end) / 100.0, 3)  # from the previous call's last exit
        rows.append(row)
        log(f"bench: spans {c.name} M={c.M}: gap {row['gap_us']} us, span {row['span_us']} us, start spread {row['start_spread_us']}, "
            f"prologue {row['prologue_us']} (args {row['args_us']}, setup {row['setup_us']}, issue {row['issue_us']}; "
            f"max {row['prologue_max_us']}), loop {row['loop_us']} "
            f"(max {row['loop_max_us']}), tail {row['tail_us']} (max {row['tail_max_us']}), {row['clock_GHz']} GHz")
    return rows


def measure(args, wl, device, steps, warmup):
    """Build workload ``wl``, capture one step in a graph (or replay eagerly), time
    ``steps`` steps after ``warmup`` between two synchronisations.  Returns the
    result fields, the per-pass calls and the config."""
    sub = argparse.Namespace(**vars(args))
    sub.workload = wl
    calls, cfg = build_workload(sub, device)
    log(f"bench: {wl}: {len(calls)} calls per pass built")
    # A captured graph replays fixed weight copies.  When one pass over the calls
    # streams less than 1.25x the Infinity Cache, a step is several passes (each on
    # the next copies), so that every replay reads its weights from HBM.
    pass_bytes = sum(c.wbytes for c in calls)
    passes = 1
    if wl not in ("prefill", "copy") and pass_bytes < MALL_BYTES * 1.25:
        passes = -(-int(MALL_BYTES * 1.25) // pass_bytes)
    cfg["passes_per_step"] = passes
    pass_calls = calls
    calls = calls * passes
    if args.eager:
        class Eager:
            def replay(self):
                for c in calls:
                    c()
        g = Eager()
    else:
        g = graph_of(calls)
        cycled = {}
        for c in pass_calls:
            if getattr(c, "wset", None) is not None and c.name not in cycled:
                cycled[c.name] = c.wset.used
        if cycled and wl not in ("stack", "stack_native"):
            cfg["weight_copies_cycled"] = cycled
            cfg["cycled_weight_bytes_per_step"] = sum(c.wbytes for c in calls)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        g.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    launches = steps * len(calls)
    res = {"steps": steps, "warmup": warmup, "ms_per_step": round(wall * 1e3 / steps, 4),
           "gpu_ms_per_step": round(gpu_ms / steps, 4),
           "gbps": sum(c.wbytes for c in calls) * steps / (gpu_ms * 1e6),
           "kb_gbps": sum(c.kb_bytes for c in calls) * steps / (gpu_ms * 1e6),
           "tflops": sum(c.flops for c in calls) * steps / (gpu_ms * 1e9),
           "avg_launch_us": gpu_ms * 1e3 / launches,
           "bytes_per_launch": sum(c.wbytes for c in calls) / len(calls)}
    log(f"bench: {wl}: timed {steps} steps: wall {wall * 1e3:.3f} ms, gpu {gpu_ms:.3f} ms")
    del g
    return res, pass_calls, cfg


def roofline_of(wl, res, calls):
    if wl == "prefill":
        roof = {"bound": "mfma", "achieved": round(res["tflops"], 1), "peak": SPARSE_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(res["tflops"] / SPARSE_F16_PEAK_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "achieved": round(res["gbps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(res["gbps"] / HBM_PEAK_GBS, 4)}
    roof["traffic"] = None
    roof["kernel"] = "device copy (calibration)" if wl == "copy" else " + ".join(sorted({kernel_of(c) for c in calls}))
    roof["avg_launch_us"] = round(res["avg_launch_us"], 3)
    roof["algorithmic_bytes_per_launch"] = round(res["bytes_per_launch"])
    return roof


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="decode",
                   choices=["decode", "decode70b", "native", "native70b", "prefill", "w3", "meta3", "dense", "stack",
                            "stack_native", "copy", "compare", "floor", "floor70b", "mfma_floor", "spans", "spans70b",
                            "spans_sweep"])
    p.add_argument("--eager", action="store_true", help="replay the calls without a HIP graph")
    p.add_argument("--prefill-m", type=int, nargs="+", default=[512, 1024, 2048, 4096])
    p.add_argument("--no-prefill", action="store_true",
                   help="decode workload: skip the prefill half of the metric (Llama-2-70B, M >= 512)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-per-call", action="store_true")
    args = p.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        raise SystemExit("bench.py measures one GPU: the 2:4 GEMM has no multi-GPU path in this build "
                         "(each GPU would own whole 64-column chunks of N, with no communication). "
                         "Run with --gpus 1.")
    if not torch.cuda.is_available():
        raise SystemExit("no GPU visible")
    if args.workload.startswith("spans"):
        from csed499ii_amd import build as _build

        _lib.LIB_PATH = _build.SPANS_LIB  # the measurement build (per-wave stamps)
    _lib.load()
    device = "cuda:0"
    log(f"bench: workload={args.workload} steps={args.steps} warmup={args.warmup}")
    base = {"metric": METRIC, "n_gpus": 1, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16", "data": "synthetic"}
    if args.workload == "compare":
        rows = compare_libraries(device)
        dec = [r for r in rows if r["M"] <= 32]
        wb = sum(synth.weight_bytes(r["K"], r["N"], 4, 128) for r in dec)
        us = sum(r["ours_us"] for r in dec)
        print(json.dumps({**base, "value": round(wb / (us * 1e3), 2), "unit": "GB/s", "steps": 0, "warmup": 0,
                          "ms_per_step": round(us / 1e3, 4),
                          "config": {"workload": "library_comparison",
                                     "note": "per call site, graph-replayed where capturable; value = this "
                                             "library's decode call sites (M in {1, 16}) on weight bytes"},
                          "compare": rows}), flush=True)
        return
    if args.workload == "mfma_floor":
        rows = mfma_floor_workload(args, device)
        fl = sum(2 * r["M"] * r["K"] * r["N"] for r in rows)
        su = sum(r["stream_us"] for r in rows)
        gu = sum(r["gemm_us"] for r in rows)
        print(json.dumps({**base, "value": round(fl / (su * 1e6), 1), "unit": "TFLOP/s", "steps": 0, "warmup": 0,
                          "ms_per_step": round(su / 1e3, 4),
                          "config": {"workload": "prefill_sweep_llama2_70b_mfma_floor",
                                     "note": "per prefill-sweep call: the MFMA-only smfmac 32x32x32 stream on its "
                                             "planned grid with the call's smfmac count, reference timing "
                                             "protocol; value = the sweep's dense-equivalent FLOPs over the summed "
                                             "stream times",
                                     "gemm_TFLOPs": round(fl / (gu * 1e6), 1)},
                          "per_call": rows}), flush=True)
        return
    if args.workload in ("floor", "floor70b"):
        rows = floor_workload(args, device, shapes_70b=args.workload == "floor70b")
        wb = sum(synth.weight_bytes(r["K"], r["N"], 4, 128) for r in rows)
        read_us = sum(r["read_us"] for r in rows)
        print(json.dumps({**base, "value": round(wb / (read_us * 1e3), 2), "unit": "GB/s", "steps": 0,
                          "warmup": 0, "ms_per_step": round(read_us / 1e3, 4),
                          "config": {"workload": "decode_sweep_llama2_%s_floor" % (
                                         "70b" if args.workload == "floor70b" else "7b"),
                                     "note": "per decode-sweep call: a plain streaming read of its weight bytes "
                                             "(best of 256-2048 workgroups, grid-stride order or a contiguous "
                                             "range per wave: read_blocks < 0) and an empty kernel on its planned "
                                             "grid, reference timing protocol; value = the sweep's weight bytes "
                                             "over the summed read times",
                                     "empty_us_sum": round(sum(r["empty_us"] for r in rows), 3)},
                          "per_call": rows}), flush=True)
        return
    if args.workload.startswith("spans"):
        rows = spans_workload(args, device, shapes_70b=args.workload == "spans70b",
                              in_sweep=args.workload == "spans_sweep")
        span = sum(r["span_us"] for r in rows)
        wb = sum(synth.weight_bytes(r["K"], r["N"], 4, 128) for r in rows)
        print(json.dumps({**base, "value": round(wb / (span * 1e3), 2), "unit": "GB/s", "steps": 0, "warmup": 0,
                          "ms_per_step": round(span / 1e3, 4),
                          "config": {"workload": "decode_sweep_llama2_%s_spans" % ("70b" if "70" in args.workload
                                                                                  else "7b"),
                                     "library": _lib.LIB_PATH.name,
                                     "note": "per decode-sweep call: per-wave phase stamps of the last call of a "
                                             "graph of 40; value = weight bytes over the summed spans (first "
                                             "wave entry to last wave exit)"},
                          "per_call": rows}), flush=True)
        return
    res, pass_calls, cfg = measure(args, args.workload, device, args.steps, args.warmup)
    wl = args.workload
    roof = roofline_of(wl, res, pass_calls)
    roof["traffic"] = traffic_from_profile(cfg["workload"])
    roof["traffic_unit"] = "bytes per launch"
    roof["ceiling"] = ceiling_from_profile(cfg["workload"], roof["achieved"])
    value, unit = (res["tflops"], "TFLOP/s") if wl == "prefill" else (res["gbps"], "GB/s")
    out = {**base, "value": round(value, 2), "unit": unit, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": res["ms_per_step"], "config": cfg, "roofline": roof,
           "kb_bench_GBps": round(res["kb_gbps"], 1)}
    if not args.no_per_call and wl != "copy":
        log("bench: per-call timing")
        out["per_call"] = per_call_stats(pass_calls if not wl.startswith("stack") else pass_calls[:4])
    if wl == "decode" and not args.no_prefill:
        # the prefill half of the metric: Llama-2-70B shapes at M >= 512, TFLOP/s
        # 10 steps (~70 ms) after 3 warm-up steps: fewer read ~2 % low from run to run
        pres, pcalls, pcfg = measure(args, "prefill", device, max(10, args.steps // 2), 3)
        proof = roofline_of("prefill", pres, pcalls)
        proof["ceiling"] = ceiling_from_profile(pcfg["workload"], proof["achieved"])
        out["prefill"] = {"value": round(pres["tflops"], 1), "unit": "TFLOP/s", "steps": pres["steps"],
                          "warmup": pres["warmup"], "ms_per_step": pres["ms_per_step"],
                          "gpu_ms_per_step": pres["gpu_ms_per_step"], "config": pcfg, "roofline": proof}
        if not args.no_per_call:
            log("bench: prefill per-call timing")
            out["prefill"]["per_call"] = per_call_stats(pcalls, samples=5, replays=2, reps=4)
        del pcalls
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline and wl in ("decode", "decode70b", "meta3", "w3", "stack", "stack_native"):
        log("bench: cpu baseline (reference CPU path)")
        out["cpu_baseline"] = cpu_baseline()
    elif not args.no_cpu_baseline:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
