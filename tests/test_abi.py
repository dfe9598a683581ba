"""The C-ABI library: it builds, loads without a GPU, exports every symbol that
include/marlin_hip.h declares, and its host-side validation returns the
reference's error codes (no kernel launch happens on these paths)."""
import ctypes
import pathlib
import re
import subprocess

import pytest

from csed499ii_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "marlin_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(marlin_hip_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "marlin_hip_mul_2_4" in syms and "marlin_hip_last_error" in syms
    assert set(syms) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(built_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT\s+(marlin_hip_\w+)", out))
    for sym in declared_symbols():
        assert sym in exported, sym
        assert hasattr(built_lib, sym)


def _mul(lib, prob_m, prob_n, prob_k, groupsize, thread_k=-1, thread_m=-1):
    null = ctypes.c_void_p(0)
    return lib.marlin_hip_mul_2_4(null, null, null, null, null, prob_m, prob_n, prob_k, null, groupsize, 0, null,
                                  thread_k, thread_m, -1, 16)


@pytest.mark.parametrize("args,expected", [
    # (prob_m=N, prob_n=batch, prob_k=K, groupsize, thread_k, thread_m)
    ((512, 16, 1024, -1, 128, 100), _lib.ERR_PROB_SHAPE),   # N % thread_m
    ((512, 16, 1000, -1, -1, -1), _lib.ERR_PROB_SHAPE),     # K % 128 (auto tile for batch <= 16)
    ((384, 32, 1024, 64, -1, -1), _lib.ERR_PROB_SHAPE),     # N % 256 (auto tile for batch > 16)
    ((512, 32, 1024, -1, 128, 128), _lib.ERR_KERN_SHAPE),   # 128x128 tile only for one batch block
    ((512, 16, 1024, -1, 256, 512), _lib.ERR_KERN_SHAPE),   # no such tile
    ((512, 16, 1024, 32, -1, -1), _lib.ERR_KERN_SHAPE),     # group_blocks 2 not instantiated
    ((512, 16, 1024, -1, 0, 0), _lib.ERR_KERN_SHAPE),       # degenerate tile
    ((0, 16, 1024, -1, -1, -1), _lib.OK),                   # empty problem: nothing to do
    ((512, 0, 1024, -1, -1, -1), _lib.OK),
])
def test_host_validation_codes(built_lib, args, expected):
    prob_m, prob_n, prob_k, g, tk, tm = args
    assert _mul(built_lib, prob_m, prob_n, prob_k, g, tk, tm) == expected


def test_codec_argument_checks(built_lib):
    null = ctypes.c_void_p(0)
    assert built_lib.marlin_hip_meta3_pack(null, null, 100, null, 0, null) == _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_meta3_unpack(null, null, 47, 0, null) == _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_expand3(null, null, -1, 0, null) == _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_meta3_pack(null, null, 0, null, 0, null) == _lib.OK


def test_native_host_validation(built_lib):
    """Shapes the native layout cannot hold are refused before any launch; an empty
    batch is a no-op."""
    null = ctypes.c_void_p(0)
    assert built_lib.marlin_hip_native_pack(null, null, null, null, null, null, 96, 512, 64, 0, null) == \
        _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_native_unpack(null, null, null, null, null, null, 128, 384, 64, 0, null) == \
        _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_mul_2_4_native(null, null, null, null, null, 128, 1, 512, 32, 0, null, -1) == \
        _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_mul_2_4_native(null, null, null, null, null, 128, 0, 512, 64, 0, null, -1) == \
        _lib.OK


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """There is no CPU fallback: without the built library every entry point raises."""
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libmarlin_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_plan_without_gpu(built_lib):
    """marlin_hip_plan is host-only: the decode sweep's plans (the split-K choices that
    decide which calls use a stream's scratch), the large-M kernel at prefill sizes,
    and the no-allocation variant, which never splits K."""
    from csed499ii_amd import marlin

    p = marlin.plan_2_4(1, 4096, 4096)
    assert p["kernel"] == "decode" and p["splits"] == 1 and p["launches"] == 1
    assert p["workgroups"] * (p["threads"] // 64) > 0
    p = marlin.plan_2_4(16, 4096, 22016, sms=256)  # 344 tiles: the 88 past one per CU split in two
    assert p["splits"] == 2 and p["workgroups"] == 256 + 2 * 88
    p = marlin.plan_2_4(24, 4096, 22016, sms=256)  # wide N above 16 rows: the 88 tail tiles split in two
    assert p["kernel"] == "decode_dma" and p["splits"] == 2 and p["workgroups"] == 256 + 2 * 88
    # 1-8 padded rows run the register-ring decode kernel, 16 and 32 the LDS-DMA one
    # (7B o at 8 rows takes the 8-row batch; 7B qkv at 8 rows the 16-row batch)
    assert [marlin.plan_2_4(M, 4096, 4096)["kernel"] for M in (1, 4, 8, 9, 16, 32)] == \
        ["decode"] * 3 + ["decode_dma"] * 3
    assert marlin.plan_2_4(8, 4096, 12288)["kernel"] == "decode_dma"
    assert marlin.plan_2_4(24, 4096, 22016, noalloc=True)["splits"] == 1
    assert marlin.plan_2_4(4, 8192, 8192)["splits"] == 1  # 16-column tiles fill the CUs
    assert marlin.plan_2_4(4, 8192, 10240)["splits"] == 4  # long K, wider N: the tail tiles split four ways
    p = marlin.plan_2_4(64, 4096, 4096)  # below the large-M threshold: two decode launches of 32 rows
    assert p["kernel"] == "decode_dma" and p["launches"] == 2
    for M in (512, 4096):
        p = marlin.plan_2_4(M, 8192, 57344)
        assert p["kernel"] == "large_m" and p["threads"] == 512
        assert p["workgroups"] == 57344 // 512 * (M // 128) * p["splits"]
    # few tiles: 64-row tiles (qkv: 160 of them), and split K (o: two ways)
    p = marlin.plan_2_4(512, 8192, 10240, sms=256)
    assert p["kernel"] == "large_m" and p["splits"] == 1 and p["workgroups"] == 10240 // 512 * (512 // 64)
    p = marlin.plan_2_4(512, 8192, 8192, sms=256)
    assert p["splits"] == 2 and p["workgroups"] == 2 * 8192 // 512 * (512 // 64)
    assert marlin.plan_2_4(512, 28672, 8192, sms=256)["splits"] == 4  # long K: 128-row tiles split four ways
    assert marlin.plan_2_4(512, 8192, 8192, noalloc=True)["splits"] == 1
    assert marlin.plan_2_4(300, 4096, 768)["kernel"] == "general"  # N % 512 != 0
    with pytest.raises(RuntimeError, match="not compatible"):
        marlin.plan_2_4(16, 1000, 512)


def test_plan_three_tiles_per_workgroup(built_lib):
    """Three 16-column tiles per workgroup of 12 waves where a third of the tiles fits
    the CUs (one workgroup per CU) and the tiles are a multiple of 96: Llama-2-7B qkv
    (768 tiles) at 1-4 rows on 256 or 304 CUs; not at 5+ rows (16-row batch or
    64-column tiles), not where 256 workgroups exceed the CUs, and not for shapes
    whose tiles are no multiple of 96 (7B o: 256 tiles)."""
    from csed499ii_amd import marlin

    for sms in (256, 304):
        for M in (1, 2, 3, 4):
            p = marlin.plan_2_4(M, 4096, 12288, sms=sms)
            assert (p["kernel"], p["workgroups"], p["threads"], p["splits"]) == ("decode", 256, 768, 1), (sms, M, p)
    assert marlin.plan_2_4(5, 4096, 12288, sms=256)["threads"] != 768
    assert marlin.plan_2_4(1, 4096, 12288, sms=80)["threads"] != 768
    assert marlin.plan_2_4(4, 4096, 12288, sms=80)["threads"] != 768
    for M in (1, 2, 4):
        assert marlin.plan_2_4(M, 4096, 4096, sms=256)["threads"] != 768
    assert marlin.plan_2_4(1, 4096, 12288, sms=256, noalloc=True)["threads"] == 768  # unsplit anyway
    assert marlin.plan_2_4(0, 4096, 4096)["kernel"] is None


def test_noalloc_host_validation(built_lib):
    """The no-allocation entry point refuses what mul_2_4 refuses, before any launch."""
    null = ctypes.c_void_p(0)
    assert built_lib.marlin_hip_mul_2_4_noalloc(null, null, null, null, null, 512, 16, 1000, -1, 0, null, -1, -1,
                                                -1) == _lib.ERR_PROB_SHAPE
    assert built_lib.marlin_hip_mul_2_4_noalloc(null, null, null, null, null, 512, 32, 1024, -1, 0, null, 128, 128,
                                                -1) == _lib.ERR_KERN_SHAPE
    assert built_lib.marlin_hip_mul_2_4_noalloc(null, null, null, null, null, 512, 0, 1024, -1, 0, null, -1, -1,
                                                -1) == _lib.OK


def test_probe_library_exports(built_lib):
    """bench.py's measurement library exports what include/marlin_probe.h declares."""
    from csed499ii_amd import build

    header = (HEADER.parent / "marlin_probe.h").read_text()
    declared = set(re.findall(r"^\s*int\s+(marlin_probe_\w+)\s*\(", header, re.M))
    assert declared == {"marlin_probe_read", "marlin_probe_empty", "marlin_probe_mfma_32x32x16", "marlin_probe_smfmac_stream"}
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.PROBE_LIB)], capture_output=True, text=True,
                         check=True).stdout
    assert declared <= set(re.findall(r"\bT\s+(marlin_probe_\w+)", out))


@pytest.mark.parametrize("args,expected", [
    # dense (prob_m = batch, prob_n = N, prob_k = K, groupsize in dense K, thread_k, thread_n)
    ((16, 512, 1024, -1, 128, 100), _lib.ERR_PROB_SHAPE),   # N % thread_n
    ((16, 512, 1000, -1, -1, -1), _lib.ERR_PROB_SHAPE),     # K % 128 (auto tile for batch <= 16)
    ((32, 384, 1024, 128, -1, -1), _lib.ERR_PROB_SHAPE),    # N % 256 (auto tile above 16 rows)
    ((32, 512, 1024, -1, 128, 128), _lib.ERR_KERN_SHAPE),   # 128x128 only for one 16-row block
    ((16, 512, 1024, 64, -1, -1), _lib.ERR_KERN_SHAPE),     # group_blocks 4 not instantiated
    ((0, 512, 1024, -1, -1, -1), _lib.OK),                  # empty problem
])
def test_dense_host_validation_codes(built_lib, args, expected):
    """marlin_hip_mul refuses shapes with the reference dispatch's codes
    (marlin_cuda_kernel.cu:660-683, 711-721) before any launch."""
    m, n, k, g, tk, tn = args
    null = ctypes.c_void_p(0)
    assert built_lib.marlin_hip_mul(null, null, null, null, m, n, k, null, g, 0, null, tk, tn, -1, 16) == expected


def test_spans_hook(built_lib):
    """The measurement hook of include/marlin_spans.h: exported by the product library
    (which records no stamps: code 2) and by the measurement build (code 0); setting
    it launches nothing, so this runs without a GPU."""
    from csed499ii_amd import build

    header = (HEADER.parent / "marlin_spans.h").read_text()
    assert re.findall(r"^\s*int\s+(marlin_hip_\w+)\s*\(", header, re.M) == ["marlin_hip_set_spans"]
    fn = built_lib.marlin_hip_set_spans
    fn.restype, fn.argtypes = ctypes.c_int, [ctypes.c_void_p]
    assert fn(None) == _lib.ERR_KERN_SHAPE
    spans = ctypes.CDLL(str(build.SPANS_LIB))
    spans.marlin_hip_set_spans.restype, spans.marlin_hip_set_spans.argtypes = ctypes.c_int, [ctypes.c_void_p]
    assert spans.marlin_hip_set_spans(None) == _lib.OK
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.SPANS_LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT\s+(marlin_hip_\w+)", out))
    assert set(declared_symbols()) <= exported


READELF = "/opt/rocm/lib/llvm/bin/llvm-readelf"


def _code_objects(lib_path):
    """The gfx950 code objects (bytes) in the offload bundles of a HIP shared
    library's .hip_fatbin section."""
    import struct

    if not pathlib.Path(READELF).exists():
        pytest.skip("llvm-readelf not available")
    hdr = subprocess.run([READELF, "-S", "--wide", str(lib_path)], capture_output=True, text=True, check=True).stdout
    m = re.search(r"\.hip_fatbin\s+PROGBITS\s+[0-9a-f]+\s+([0-9a-f]+)\s+([0-9a-f]+)", hdr)
    assert m, "no .hip_fatbin section"
    off, size = int(m.group(1), 16), int(m.group(2), 16)
    data = pathlib.Path(lib_path).read_bytes()[off:off + size]
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    pos = 0
    while (i := data.find(magic, pos)) >= 0:
        n = struct.unpack_from("<Q", data, i + 24)[0]
        p = i + 32
        for _ in range(n):
            eo, es, ts = struct.unpack_from("<QQQ", data, p)
            triple = data[p + 24:p + 24 + ts].decode()
            p += 24 + ts
            if "gfx950" in triple:
                yield data[i + eo:i + eo + es]
        pos = i + len(magic)


def _kernel_scratch(lib_path):
    """{kernel symbol: private segment bytes} of every gfx950 kernel in a HIP shared
    library: each code object's metadata note read with llvm-readelf."""
    import tempfile

    out = {}
    for co in _code_objects(lib_path):
        with tempfile.NamedTemporaryFile(suffix=".co") as f:
            f.write(co)
            f.flush()
            notes = subprocess.run([READELF, "--notes", f.name], capture_output=True, text=True, check=True).stdout
        for name, priv in re.findall(r"\.name:\s+(\S+)\n(?:.*\n)*?\s+\.private_segment_fixed_size:\s+(\d+)",
                                     notes):
            out[name] = int(priv)
    return out


def _kernarg_preload(lib_path):
    """{kernel symbol: kernel-argument dwords preloaded into SGPRs} of every gfx950
    kernel of a HIP shared library, from its kernel descriptor (the 64-byte `.kd`
    object: uint16 at byte 58, bits 0-6 KERNARG_PRELOAD_SPEC_LENGTH)."""
    import struct
    import tempfile

    out = {}
    for co in _code_objects(lib_path):
        with tempfile.NamedTemporaryFile(suffix=".co") as f:
            f.write(co)
            f.flush()
            secs = subprocess.run([READELF, "-S", "--wide", f.name], capture_output=True, text=True, check=True).stdout
            syms = subprocess.run([READELF, "-s", "--wide", f.name], capture_output=True, text=True, check=True).stdout
        # [Nr] Name Type Address Off Size ...: address ranges mapped to file offsets
        ranges = [(int(a, 16), int(o, 16), int(z, 16))
                  for a, o, z in re.findall(r"\]\s+\S+\s+\S+\s+([0-9a-f]{8,})\s+([0-9a-f]{6,})\s+([0-9a-f]{6,})", secs)]
        for value, name in re.findall(r"^\s*\d+:\s+([0-9a-f]+)\s+64\s+OBJECT\s+\S+\s+\S+\s+\S+\s+(\S+)\.kd$", syms,
                                      re.M):
            addr = int(value, 16)
            base = next(o + addr - a for a, o, z in ranges if a <= addr < a + z)
            out[name] = struct.unpack_from("<H", co, base + 58)[0] & 0x7F
    return out


def test_decode_kernels_preload_their_leading_arguments(built_lib):
    """The decode-sized kernels take the fields their prologue needs first as leading
    scalar arguments, built to be preloaded into SGPRs: the register-ring, LDS-DMA
    and lane-native decode kernels 14 dwords, the dense Marlin kernel 12; kernels whose
    first argument is a struct preload nothing."""
    pre = _kernarg_preload(_lib.LIB_PATH)
    fam = {"sm24_decode_kernel": 14, "sm24_decode_dma_kernel": 14, "sm24_native_decode_kernel": 14,
           "marlin_dense_kernel": 12, "sm24_prefill_kernel": 0}
    for part, want in fam.items():
        got = {k: v for k, v in pre.items() if part + "I" in k}
        assert got, part
        assert set(got.values()) == {want}, (part, sorted(set(got.values())))


def test_no_kernel_spills_to_scratch(built_lib, tmp_path):
    """No kernel of the GEMM library or of the measurement library keeps anything in
    scratch (private) memory: a spill would stream every wave's registers through
    memory.  The reader itself finds the scratch of a kernel built to need it."""
    from csed499ii_amd import build

    for lib in (_lib.LIB_PATH, build.SPANS_LIB, build.PROBE_LIB):
        sizes = _kernel_scratch(lib)
        assert len(sizes) >= (100 if lib != build.PROBE_LIB else 4), lib.name
        assert not {k: v for k, v in sizes.items() if v}, f"{lib.name}: kernels using scratch"
    src = tmp_path / "spill.hip"
    src.write_text("#include <hip/hip_runtime.h>\n"
                   "__global__ void spill_kernel(const int* i, float* o) {\n"
                   "  float a[256];\n  for (int k = 0; k < 256; k++) a[k] = o[k] * 2.f;\n"
                   "  o[threadIdx.x] = a[i[threadIdx.x] & 255];\n}\n")
    so = tmp_path / "libspill.so"
    subprocess.run([build.hipcc(), f"--offload-arch={build.ARCH}", "-O3", "-fPIC", "-shared", "-o", str(so),
                    str(src)], check=True, capture_output=True)
    assert any(v > 0 for v in _kernel_scratch(so).values())
