"""Build the gfx950 HIP library libxtu_moe_amd.so in-tree.

Each csrc/*.hip is compiled for gfx950 with hipcc and each csrc/*.cpp (host
code only: the host expert engine) with g++, in parallel, then linked into
xtu_moe_amd/lib/libxtu_moe_amd.so, which the Python package loads with
ctypes.  Packed-fp32 VALU instructions are disabled for all device code.
The test-only probe library (tests/probes/probes.hip ->
tests/probes/libxtu_probes.so) is built beside it, separately.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "xtu_moe_amd", "lib")
LIB = os.path.join(OUT_DIR, "libxtu_moe_amd.so")
OBJ_DIR = os.path.join(HERE, "_build")
PROBE_SRC = os.path.join(os.path.dirname(HERE), "tests", "probes", "probes.hip")
PROBE_LIB = os.path.join(os.path.dirname(HERE), "tests", "probes", "libxtu_probes.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


CXX = os.environ.get("CXX", "g++")
# host code: no -march (the library runs on other hosts); AVX-512 paths are
# compiled per function and chosen at run time
CXXFLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-pthread", "-fvisibility=hidden"]


# per-file device flags: the FP8 pair kernel rescales its accumulators with
# VALU multiplies, so its MFMA results live in VGPRs (no AGPR round trips)
EXTRA = {"f8pair32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    if src.endswith(".cpp"):
        cmd = [CXX, *CXXFLAGS, "-I", CSRC, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *CFLAGS, *EXTRA.get(os.path.basename(src), []), "-I", CSRC, "-c", src,
               "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the device-only target feature; that note is harmless
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed for {src}:\n{err}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with_probes = os.path.exists(PROBE_SRC)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + 1)) as ex:
        objs = list(ex.map(_compile, srcs + ([PROBE_SRC] if with_probes else [])))
    if with_probes:
        _link([objs.pop()], PROBE_LIB)
    _link(objs, LIB)
    shutil.rmtree(OBJ_DIR, ignore_errors=True)
    if verbose:
        print(f"built {LIB}" + (f" and {PROBE_LIB}" if with_probes else ""))
    return LIB


def _link(objs, out):
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {out} failed:\n{r.stderr}")
    os.replace(tmp, out)


if __name__ == "__main__":
    build()
    sys.exit(0)
