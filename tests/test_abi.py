"""C ABI: the library exports every entry point the header declares, and the
ctypes signature table matches the header argument by argument."""
import ctypes
import os
import re
import subprocess

import pytest

from xtu_moe_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "xtu_moe_amd.h")


def _prototypes():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b((?:xtu|moe4_smallm)_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        params = [] if args in ("", "void") else [a.strip() for a in args.split(",")]
        out[name] = (ret, params)
    return out


def _kind(ctype: str) -> str:
    c = " ".join(ctype.split())
    if "*" in c or "hipStream_t" in c:
        return "ptr"
    if c.startswith("float"):
        return "f32"
    if c.startswith("long"):
        return "i64"
    if c.startswith("size_t"):
        return "size"
    if c.startswith("int") or c.startswith("hipError_t") or c.startswith("const int"):
        return "i32"
    raise AssertionError(f"unmapped C type {ctype!r}")


def _ckind(t) -> str:
    return {ctypes.c_void_p: "ptr", ctypes.c_float: "f32", ctypes.c_long: "i64",
            ctypes.c_size_t: "size", ctypes.c_int: "i32", ctypes.c_char_p: "ptr"}[t]


def test_header_and_ctypes_table_agree():
    protos = _prototypes()
    assert set(protos) == set(_lib.SIGNATURES), (
        f"header-only: {set(protos) - set(_lib.SIGNATURES)}, "
        f"table-only: {set(_lib.SIGNATURES) - set(protos)}")
    for name, (ret, params) in protos.items():
        res, args = _lib.SIGNATURES[name]
        want = [_kind(" ".join(p.split()[:-1]) if p.split()[-1].lstrip("*").isidentifier() else p)
                for p in params]
        got = [_ckind(a) for a in args]
        assert want == got, f"{name}: header {want} vs ctypes {got}"


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = set(_prototypes()) - exported
    assert not missing, f"not exported: {missing}"


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_library_loads_and_reports_version():
    lib = _lib.load()
    assert _lib.version().startswith("xtu-moe-amd")
    # argument validation runs on the host: a bad shape is rejected without a launch
    rc = lib.xtu_route_softmax_topk(None, 4, 0, 2, 1, None, None, None)
    assert rc == 1   # hipErrorInvalidValue
    assert all(_lib.load().xtu_gemm_tile_m(f) == 128 for f in range(4))
    assert _lib.load().xtu_gemm_tile_m(4) == 0
    # exact-pair tiles: 64 rows (16x16x128 kernel), 128 on the MXFP4
    # 32x32x64 kernel where the shape fits it
    assert lib.xtu_gemm8_tile_m() == 64 and lib.xtu_mx_pair_tile_m() == 128
    assert lib.xtu_mx_pair_fits(7168, 2048) == 1 and lib.xtu_mx_pair_fits(2048, 768) == 1
    assert lib.xtu_mx_pair_fits(2880, 2880) == 0 and lib.xtu_mx_pair_fits(7168, 2176) == 0
    assert lib.xtu_mx_pair_fits(32768, 2048) == 0   # activation scales of 128 rows exceed LDS
    # FP8 32x32x64 kernel: 128 rows; H in 256-column down blocks, I in 128-row
    # scale blocks, activation scales of 128 rows in LDS
    assert lib.xtu_f8_pair_tile_m() == 128
    assert lib.xtu_f8_pair_fits(7168, 2048) == 1 and lib.xtu_f8_pair_fits(2048, 768) == 1
    assert lib.xtu_f8_pair_fits(2880, 2880) == 0 and lib.xtu_f8_pair_fits(7168, 2112) == 0
    assert lib.xtu_f8_pair_fits(32768, 2048) == 0


PROBE_HEADER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "probes", "xtu_probes.h")


def _exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_product_library_carries_no_test_probes():
    assert not [s for s in _exports(_lib.LIB_PATH) if s.startswith("xtu_probe")]


def test_probe_library_matches_its_header():
    from probes import probe_lib
    global HEADER
    saved, HEADER = HEADER, PROBE_HEADER
    try:
        protos = _prototypes()
    finally:
        HEADER = saved
    assert set(protos) == set(probe_lib.SIGNATURES)
    if os.path.exists(probe_lib.LIB_PATH):
        assert not set(protos) - _exports(probe_lib.LIB_PATH)
