"""ctypes binding of the test-only probe library (libxtu_probes.so, built by
vllm-xtu-moe_amd/build_lib.py from tests/probes/probes.hip; declarations in
tests/probes/xtu_probes.h)."""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libxtu_probes.so")

_vp, _i = ctypes.c_void_p, ctypes.c_int
SIGNATURES = {
    "xtu_probe_fp4": (_i, [_vp, _i, _vp, _vp]),
    "xtu_probe_fp4_mul": (_i, [_vp, _i, _vp, _vp]),
    "xtu_probe_fp8": (_i, [_vp, _vp]),
    "xtu_probe_mfma": (_i, [_i, _vp, _vp, _vp, _vp]),
    "xtu_probe_exp": (_i, [_vp, _i, _vp, _vp, _vp]),
    "xtu_probe_mfma_scaled_fp4b": (_i, [_vp, _vp, _vp, _vp, _vp, _vp]),
}
_LIB = None


def load():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (python vllm-xtu-moe_amd/build_lib.py)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _LIB = lib
    return _LIB


def call(name: str, *args):
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed: hipError {rc}")
    return rc
