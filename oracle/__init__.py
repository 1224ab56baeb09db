"""Oracle of the quantized MoE expert path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker (or the timed CPU baseline),
never as part of the product path.

Two backends:

* ``lib/libxtu_oracle.so`` -- the C restatement in ``xtu_oracle.c`` (routers,
  segmentation, codecs, expert math, INT8 ALIGN integer path);
* ``_ref/libxref_<isa>.so`` -- the reference xiaotu-moe CPU engine
  (``xiaotu_moe/csrc/moe/moe_v2.hpp`` ``MOE_V2::forward_many``) compiled from the
  reference's own headers behind ``ref_engine.cpp``.  Built only where the
  reference checkout exists; elsewhere the prebuilt file is used.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = {}

FMT_BF16, FMT_FP8, FMT_MXFP4, FMT_NVFP4, FMT_INT4 = 0, 1, 2, 3, 4


def build(force: bool = False) -> None:
    """Compile the oracle (and, where the reference checkout exists, oracle/_ref)."""
    so = os.path.join(_HERE, "lib", "libxtu_oracle.so")
    if force or not os.path.exists(so):
        subprocess.run(["bash", os.path.join(_HERE, "build_ref.sh")], check=True)


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def lib():
    global _LIB
    if _LIB is None:
        so = os.path.join(_HERE, "lib", "libxtu_oracle.so")
        if not os.path.exists(so):
            build()
        L = ctypes.CDLL(so)
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.xo_e2m1.restype = f
        L.xo_e8m0.restype = f
        L.xo_e4m3.restype = f
        L.xo_expf.restype = f
        L.xo_expf.argtypes = [f]
        L.xo_sigmoid.restype = f
        L.xo_sigmoid.argtypes = [f]
        L.xo_silu_gate.restype = f
        L.xo_silu_gate.argtypes = [f, f, f, f, f]
        L.xo_f32_to_bf16.restype = ctypes.c_uint16
        L.xo_f32_to_bf16.argtypes = [f]
        L.xo_route_softmax_topk.argtypes = [vp, i, i, i, i, vp, vp]
        L.xo_route_grouped_sigmoid.argtypes = [vp, vp, i, i, i, i, i, f, i, vp, vp]
        L.xo_segment.argtypes = [vp, vp, i, i, i, i, i, vp, vp, vp, vp, vp]
        L.xo_moe_layer.argtypes = [i] * 7 + [vp] * 9 + [f] * 3 + [vp]
        L.xo_moe_layer_g.argtypes = [i] * 8 + [vp] * 9 + [f] * 3 + [vp]
        L.xo_moe_layer_i8.argtypes = [i] * 6 + [vp] * 7 + [f] * 3 + [vp]
        L.xo_i8_gemm.argtypes = [vp, i, vp, vp, i, i, f, vp, vp]
        L.xo_i8_quant_row.argtypes = [vp, i, vp]
        _LIB = L
    return _LIB


# --------------------------------------------------------------------- codecs
def e2m1_table() -> np.ndarray:
    L = lib()
    return np.array([L.xo_e2m1(i) for i in range(16)], np.float32)


def e8m0_table() -> np.ndarray:
    L = lib()
    return np.array([L.xo_e8m0(i) for i in range(256)], np.float32)


def e4m3_table() -> np.ndarray:
    L = lib()
    return np.array([L.xo_e4m3(i) for i in range(256)], np.float32)


def expf(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.asarray(x, np.float32).ravel()
    return np.array([L.xo_expf(float(v)) for v in x], np.float32)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# -------------------------------------------------------------------- routing
def route_softmax_topk(logits: np.ndarray, K: int, renormalize: bool = True):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    ids = np.zeros((T, K), np.int32)
    wts = np.zeros((T, K), np.float32)
    rc = lib().xo_route_softmax_topk(_p(logits), T, E, K, int(renormalize), _p(ids), _p(wts))
    if rc != 0:
        raise ValueError(f"oracle softmax router: unsupported E={E} K={K}")
    return ids, wts


def route_grouped_sigmoid(logits, bias, n_group, topk_group, K, routed_scaling=1.0,
                          renormalize=True):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ids = np.zeros((T, K), np.int32)
    wts = np.zeros((T, K), np.float32)
    rc = lib().xo_route_grouped_sigmoid(_p(logits), _p(b), T, E, n_group, topk_group, K,
                                        float(routed_scaling), int(renormalize), _p(ids), _p(wts))
    if rc != 0:
        raise ValueError(f"oracle grouped router: unsupported E={E} n_group={n_group} K={K}")
    return ids, wts


# --------------------------------------------------------------- segmentation
def segment(ids: np.ndarray, wts: np.ndarray, E: int, n_shared: int = 0,
            drop_zero: bool = False) -> dict:
    ids = np.ascontiguousarray(ids, np.int32)
    wts = np.ascontiguousarray(wts, np.float32)
    T, K = ids.shape
    A = T * K + T * n_shared
    NB = E + n_shared + 1
    out = dict(
        sorted_pair=np.zeros(max(A, 1), np.int32), sorted_tok=np.zeros(max(A, 1), np.int32),
        sorted_wts=np.zeros(max(A, 1), np.float32), inv=np.zeros(max(A, 1), np.int32),
        seg_start=np.zeros(NB + 1, np.int32))
    lib().xo_segment(_p(ids), _p(wts), T, K, E, n_shared, int(drop_zero),
                     _p(out["sorted_pair"]), _p(out["sorted_tok"]), _p(out["sorted_wts"]),
                     _p(out["inv"]), _p(out["seg_start"]))
    for k in ("sorted_pair", "sorted_tok", "sorted_wts", "inv"):
        out[k] = out[k][:A]
    return out


# ---------------------------------------------------------------- expert math
def gate_up_scales2(gs13):
    """NVFP4 second-level scales of w13 as [E, 2] fp32 (gate, up): a
    per-expert [E] vector (one scale for both halves) is repeated."""
    if gs13 is None:
        return None
    g = np.asarray(gs13, np.float32)
    if g.ndim == 1:
        g = np.repeat(g[:, None], 2, axis=1)
    if g.ndim != 2 or g.shape[1] != 2:
        raise ValueError(f"gs13 must be [E] or [E, 2], got {g.shape}")
    return np.ascontiguousarray(g)


def moe_layer(fmt: int, x_bf16: np.ndarray, ids, wts, E: int, n_shared: int, H: int, I: int,
              w13, s13, w2, s2, gs13=None, gs2=None, limit=0.0, alpha=1.0, beta=0.0):
    """out[T][H] fp32 of the dequantized-fp32 layer (CPU-engine semantics).
    INT4 (fmt 4): s13 / s2 fp32 [E, N, K/group], the group read off their
    shape."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    ids = np.ascontiguousarray(ids, np.int32)
    wts = np.ascontiguousarray(wts, np.float32)
    T, K = ids.shape
    out = np.zeros((T, H), np.float32)
    gs13 = gate_up_scales2(gs13)
    arrs = [np.ascontiguousarray(a) if a is not None else None for a in (w13, s13, gs13, w2, s2, gs2)]
    gk = H // s13.shape[-1] if fmt == 4 else 0
    rc = lib().xo_moe_layer_g(fmt, gk, T, K, E, n_shared, H, I, _p(x), _p(ids), _p(wts),
                              *[_p(a) for a in arrs], float(limit), float(alpha), float(beta),
                              _p(out))
    assert rc == 0
    return out


def moe_layer_i8(x_bf16, ids, wts, E, n_shared, H, I, w13, s13, w2, s2, limit=0.0,
                 alpha=1.0, beta=0.0):
    x = np.ascontiguousarray(x_bf16, np.uint16)
    ids = np.ascontiguousarray(ids, np.int32)
    wts = np.ascontiguousarray(wts, np.float32)
    T, K = ids.shape
    out = np.zeros((T, H), np.float32)
    arrs = [np.ascontiguousarray(a) for a in (w13, s13, w2, s2)]
    rc = lib().xo_moe_layer_i8(T, K, E, n_shared, H, I, _p(x), _p(ids), _p(wts),
                               *[_p(a) for a in arrs], float(limit), float(alpha), float(beta),
                               _p(out))
    assert rc == 0
    return out


def i8_gemm(a_f32: np.ndarray, w: np.ndarray, s: np.ndarray, gs: float = 1.0):
    """INT8 ALIGN GEMM: returns (acc int32 [M][N], c fp32 [M][N], max row shift)."""
    a = np.ascontiguousarray(a_f32, np.float32)
    M, K = a.shape
    N = w.shape[0]
    w = np.ascontiguousarray(w, np.uint8)
    s = np.ascontiguousarray(s, np.uint8)
    acc = np.zeros((M, N), np.int32)
    c = np.zeros((M, N), np.float32)
    d = lib().xo_i8_gemm(_p(a), M, _p(w), _p(s), N, K, float(gs), _p(acc), _p(c))
    return acc, c, int(d)


def i8_quant_row(a_f32: np.ndarray):
    a = np.ascontiguousarray(a_f32, np.float32).ravel()
    a8 = np.zeros(a.size, np.int8)
    crow = lib().xo_i8_quant_row(_p(a), a.size, _p(a8))
    return a8, int(crow)


# ------------------------------------------------------- reference CPU engine
def ref_isa_candidates():
    """Reference-engine builds this host can run, best first."""
    flags = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = line
                    break
    except OSError:
        pass
    have = set(flags.split())
    out = []
    if {"avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512_bf16", "avx512vbmi",
            "avx512_vnni"} <= have:
        out.append("avx512_vnni")
    if {"avx512f", "avx512bw", "avx512vl", "avx512dq"} <= have:
        out.append("avx512")
    return out


def ref_available(isa: str | None = None) -> bool:
    for cand in ([isa] if isa else ref_isa_candidates()):
        if os.path.exists(os.path.join(_HERE, "_ref", f"libxref_{cand}.so")):
            return True
    return False


def ref_lib(isa: str | None = None):
    for cand in ([isa] if isa else ref_isa_candidates()):
        if cand in _REF:
            return _REF[cand]
        so = os.path.join(_HERE, "_ref", f"libxref_{cand}.so")
        if not os.path.exists(so):
            continue
        L = ctypes.CDLL(so)
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.xref_create.restype = vp
        L.xref_create.argtypes = [i] * 7 + [f] * 3 + [vp] * 6
        L.xref_forward.argtypes = [vp, i, i, vp, vp, vp, vp]
        L.xref_forward.restype = i
        L.xref_destroy.argtypes = [vp]
        L.xref_set_int8.argtypes = [i, i]
        L.xref_mxfp4_gate_up.argtypes = [i, vp, vp, vp, vp, i, i, i]
        L.xref_mxfp4_down.argtypes = [i, vp, vp, vp, vp, i, i, i]
        L.xref_isa.restype = i
        _REF[cand] = L
        return L
    raise RuntimeError("reference engine build (oracle/_ref) not available on this host")


class RefEngine:
    """The reference ``MOE_V2`` CPU engine over dense checkpoint-layout weights.

    fmt: FMT_BF16 / FMT_FP8 / FMT_MXFP4 / FMT_NVFP4 / FMT_INT4 (the engine's
    WNA16 traits; fp32 scales [E, N, K/group]).  For NVFP4 the e4m3 scale
    bytes are handed to the engine as fp32 (exact) with the per-expert global
    scale passed separately, as the engine's NVFP4 traits expect; gate and up
    scales given separately (gs13 [E, 2]) are folded into the fp32 group
    scales instead, as the reference hook does.
    """

    def __init__(self, fmt, E, K, H, I, w13, s13, w2, s2, gs13=None, gs2=None,
                 limit=0.0, alpha=1.0, beta=0.0, isa=None):
        self.L = ref_lib(isa)
        gn, gk = {FMT_BF16: (1, 1), FMT_FP8: (128, 128), FMT_MXFP4: (1, 32),
                  FMT_NVFP4: (1, 16), FMT_INT4: (1, 0)}[fmt]
        if fmt == FMT_INT4:
            gk = H // s13.shape[-1]
        if fmt == FMT_NVFP4:
            t = e4m3_table()
            s13 = t[np.asarray(s13)]
            s2 = t[np.asarray(s2)]
            if gs13 is not None and np.asarray(gs13).ndim == 2:
                # gate and up scales that may differ: folded into the fp32
                # group scales per half, as the reference hook hands them to
                # its NVFP4 engine (hybrid_model.py:1546-1563)
                g13 = np.asarray(gs13, np.float32)
                s13 = s13.copy()
                s13[:, :I] *= g13[:, 0, None, None]
                s13[:, I:] *= g13[:, 1, None, None]
                s2 = s2 * np.asarray(gs2, np.float32)[:, None, None]
                gs13 = np.ones(E, np.float32)
                gs2 = np.ones(E, np.float32)
        self._keep = [np.ascontiguousarray(a) if a is not None else None
                      for a in (w13, w2, s13, s2, gs13, gs2)]
        k = self._keep
        self.h = self.L.xref_create(fmt, E, K, H, I, gn, gk, float(limit), float(alpha),
                                    float(beta), _p(k[0]), _p(k[1]), _p(k[2]), _p(k[3]),
                                    _p(k[4]), _p(k[5]))
        if not self.h:
            raise RuntimeError("xref_create failed")
        self.H = H

    def forward(self, x_bf16, ids, wts, out=None):
        x = np.ascontiguousarray(x_bf16, np.uint16)
        ids = np.ascontiguousarray(ids, np.uint32)
        wts = np.ascontiguousarray(wts, np.float32)
        M, K = ids.shape
        if out is None:
            out = np.zeros((M, self.H), np.float32)
        rc = self.L.xref_forward(self.h, M, K, _p(ids), _p(wts), _p(x), _p(out))
        assert rc == 0
        return out

    def close(self):
        if self.h:
            self.L.xref_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass
