"""ctypes binding of ``libmarlin_hip.so`` (C ABI declared in ``include/marlin_hip.h``).

The library is built in-tree by ``python -m csed499ii_amd.build``.  There is no
fallback: when the library is missing every GPU entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading

#: The in-tree build; MARLIN_HIP_LIB names another build of the same library (read
#: once, at import).
LIB_PATH = pathlib.Path(os.environ.get("MARLIN_HIP_LIB") or
                        pathlib.Path(__file__).resolve().with_name("libmarlin_hip.so"))

OK = 0
ERR_PROB_SHAPE = 1
ERR_KERN_SHAPE = 2
ERR_LAUNCH = 3

_vp = ctypes.c_void_p
_i = ctypes.c_int
_ll = ctypes.c_longlong

#: name -> (restype, argtypes); must match include/marlin_hip.h
SIGNATURES = {
    "marlin_hip_mul_2_4": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _i, _i, _i, _i]),
    "marlin_hip_mul_2_4_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i, _i, _i]),
    "marlin_hip_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_i)]),
    "marlin_hip_mul": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _i, _i, _i, _i]),
    "marlin_hip_mul_2_4_meta3": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _i, _i, _i, _i]),
    "marlin_hip_mul_2_4_w3": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _i, _i, _i, _i]),
    "marlin_hip_meta3_pack": (_i, [_vp, _vp, _ll, _vp, _i, _vp]),
    "marlin_hip_meta3_unpack": (_i, [_vp, _vp, _ll, _i, _vp]),
    "marlin_hip_expand3": (_i, [_vp, _vp, _ll, _i, _vp]),
    "marlin_hip_native_pack": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "marlin_hip_native_unpack": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "marlin_hip_mul_2_4_native": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i]),
    "marlin_hip_last_error": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once and set the argument types of every export."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m csed499ii_amd.build` "
                    "(there is no CPU fallback for the 2:4 GEMM)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


def last_error() -> str:
    msg = load().marlin_hip_last_error()
    return msg.decode() if msg else ""
