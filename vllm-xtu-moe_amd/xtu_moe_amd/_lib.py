"""ctypes binding of libxtu_moe_amd.so (the gfx950 HIP library).

The library is the product path: there is no fallback.  Loading fails loudly
when the shared object is missing or a symbol is absent, and every call
raises ``RuntimeError`` on a non-zero hipError_t.  Device pointers and
streams cross as integers (``tensor.data_ptr()``, ``stream.cuda_stream``).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libxtu_moe_amd.so")

_vp, _i, _l, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); hipError_t returns are checked by `call`
SIGNATURES = {
    "xtu_version": (ctypes.c_char_p, []),
    "xtu_error_string": (ctypes.c_char_p, [_i]),
    "xtu_route_softmax_topk": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "xtu_route_grouped_sigmoid": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _vp]),
    "xtu_route_segment_small_max_pairs": (_i, []),
    "xtu_route_segment_small": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp, _i,
                                     _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp]),
    "xtu_segment_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "xtu_segment_max_tiles": (_i, [_i, _i, _i, _i, _i]),
    "xtu_segment": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                         _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "xtu_segment_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp,
                                 _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "xtu_decode_gate_up": (_i, [_i, _vp, _i, _i, _i, _vp, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                                _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_decode_down": (_i, [_i, _vp, _i, _i, _i, _vp, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                             _vp, _i, _vp, _vp]),
    "xtu_decode_down_by_pair": (_i, [_i, _vp, _i, _i, _i, _vp, _vp, _vp, _l, _l, _vp, _vp, _vp,
                                     _vp, _vp, _i, _vp, _vp, _vp]),
    "xtu_combine_by_pair": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "xtu_decode_down_combine_ok": (_i, [_i, _i, _i, _i, _i, _i, _i, _i]),
    "xtu_decode_down_combine": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _l, _l,
                                     _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _i, _vp]),
    "xtu_decode_route_shared_ok": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _i]),
    "xtu_decode_route_shared": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp,
                                     _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _i, _vp, _i, _i, _vp, _vp, _vp, _l, _l, _vp,
                                     _vp, _f, _f, _f, _vp]),
    "xtu_decode_route_gate_up_ok": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _i]),
    "xtu_decode_route_gate_up": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp,
                                      _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _i, _vp, _i, _i, _vp, _vp, _vp, _l, _l, _vp,
                                      _i, _vp, _vp, _f, _f, _f, _vp]),
    "xtu_decode_layer_barrier_words": (_i, []),
    "xtu_decode_layer_ok": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _i]),
    "xtu_decode_layer": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp,
                              _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                              _vp, _vp, _i, _vp, _i, _i, _vp, _vp, _vp, _l, _l, _vp,
                              _i, _vp, _vp, _f, _f, _f, _vp, _vp, _vp, _l, _l, _vp, _i, _vp,
                              _vp]),
    "xtu_decode_gate_up_routed": (_i, [_i, _vp, _i, _i, _i, _vp, _vp, _vp, _l, _l, _vp, _vp,
                                       _vp, _vp, _vp, _vp, _i, _i, _vp, _f, _f, _f, _vp]),
    "xtu_gemm_tile_m": (_i, [_i]),
    "xtu_gemm_gate_up": (_i, [_i, _vp, _vp, _i, _i, _vp, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                              _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_gemm_down": (_i, [_i, _vp, _i, _i, _vp, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp, _vp, _vp,
                           _i, _vp, _vp]),
    "xtu_combine": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "xtu_gemm8_tile_m": (_i, []),
    "xtu_mx_pair_fits": (_i, [_i, _i]),
    "xtu_mx_pair_tile_m": (_i, []),
    "xtu_pair_quant_il": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "xtu_mx_pair_scales": (_i, [_vp, _i, _i, _i, _l, _vp, _vp]),
    "xtu_mx_pair_gate_up": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                                 _vp, _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_mx_pair_down": (_i, [_vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp, _vp, _vp,
                              _vp, _i, _vp, _vp]),
    "xtu_tri_quant_il": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "xtu_mx_tri_gate_up": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                                _vp, _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_mx_tri_down": (_i, [_vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp, _vp, _vp,
                             _vp, _i, _vp, _vp]),
    "xtu_mx_gate_up_q": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                              _vp, _vp, _vp, _i, _vp, _vp, _f, _f, _f, _vp]),
    "xtu_f8_pair_gate_up_q": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _vp, _i, _vp, _vp, _f, _f, _f, _vp]),
    "xtu_mx_duo_gate_up": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                                _vp, _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_mx_duo_down": (_i, [_vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp, _vp, _vp,
                             _vp, _i, _vp, _vp]),
    "xtu_fp8pair_quant": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "xtu_gemm8_gate_up": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp,
                               _vp, _vp, _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_gemm8_down": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp, _vp,
                            _vp, _vp, _i, _vp, _vp]),
    "xtu_gemm_pair_gate_up": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_gemm_pair_down": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp,
                                _vp, _vp, _vp, _vp, _i, _vp, _vp]),
    "xtu_copy_experts": (_i, [_i, _vp, _vp, _l, _vp, _l, _l, _vp]),
    "xtu_copy_2d": (_i, [_vp, _sz, _vp, _sz, _sz, _sz, _vp]),
    "xtu_i8_weight_bytes": (_sz, [_i, _i]),
    "xtu_i8_prepare": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "xtu_i8_quant_rows": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "xtu_i8_gemm_gate_up": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _i, _vp, _vp, _f, _f, _f, _vp]),
    "xtu_i8_gemm_down": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                              _vp, _vp]),
    "xtu_f8_pair_fits": (_i, [_i, _i]),
    "xtu_f8_pair_tile_m": (_i, []),
    "xtu_f8_pair_gate_up": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp,
                                 _vp, _vp, _vp, _i, _vp, _f, _f, _f, _vp]),
    "xtu_f8_pair_down": (_i, [_vp, _vp, _i, _i, _vp, _vp, _l, _l, _vp, _vp, _vp, _vp, _vp, _vp,
                              _vp, _i, _vp, _vp]),
    "moe4_smallm_init": (_i, []),
    "moe4_smallm_gu": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "moe4_smallm_dn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "moe4_smallm_gu2": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "moe4_smallm_dn2": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "xtu_pin_split": (_i, [_vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "xtu_cpu_engine_create": (_i, [_i, _i, _i, _i, _i, _vp, _l, _vp, _l, _vp, _l, _vp, _l, _vp,
                                   _vp, _i, _f, _f, _f, _i, _i, _i, _i, _vp]),
    "xtu_cpu_engine_info": (_i, [_vp, _vp, _vp]),
    "xtu_cpu_forward": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "xtu_cpu_decode": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "xtu_cpu_engine_destroy": (_i, [_vp]),
    "xtu_i8_fallback": (_i, [_i, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i,
                             _vp, _vp, _vp, _f, _f, _f, _vp]),
    "xtu_i8_emin_min": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "xtu_i8_row_fallback": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _vp, _vp, _i, _i, _vp, _f, _f, _f, _vp]),
}

# entry points whose int return value is a size/count, not a status
_NOT_STATUS = {"xtu_version", "xtu_error_string", "xtu_segment_workspace_bytes",
               "xtu_route_segment_small_max_pairs",
               "xtu_segment_max_tiles", "xtu_gemm_tile_m", "xtu_gemm8_tile_m",
               "xtu_mx_pair_fits", "xtu_mx_pair_tile_m", "xtu_f8_pair_fits",
               "xtu_f8_pair_tile_m",
               "xtu_decode_down_combine_ok", "xtu_decode_route_shared_ok",
               "xtu_decode_route_gate_up_ok", "xtu_decode_layer_ok",
               "xtu_decode_layer_barrier_words",
               "xtu_i8_weight_bytes"}

_LIB = None


def load():
    """Load the library (once).  Raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libxtu_moe_amd.so not found at {LIB_PATH}; build it with "
            "`python vllm-xtu-moe_amd/build_lib.py` (the HIP library is required, "
            "there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)   # AttributeError here = stale build
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)


def call(name: str, *args):
    """Call an entry point; raise on a non-zero hipError_t."""
    fn = getattr(load(), name)
    rc = fn(*args)
    if name not in _NOT_STATUS and rc != 0:
        msg = load().xtu_error_string(int(rc))
        raise RuntimeError(f"{name} failed: hipError {rc} ({msg.decode() if msg else '?'})")
    return rc


def version() -> str:
    return load().xtu_version().decode()
