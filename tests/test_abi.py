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
