"""Builds libmicro_engram_amd.so (the HIP kernels + C-ABI) in-tree for gfx950.

Each csrc/*.hip compiles to an object under csrc/_build/ in parallel, then hipcc links the
shared library next to this file. Every call compiles again (a build check must not trust a
stale library).
"""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ_DIR = os.path.join(CSRC, "_build")
LIB_NAME = "libmicro_engram_amd.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
# calibration kernels of the benchmark (csrc/calib/*.hip): a library of their own, loaded by
# bench.py only
CALIB_DIR = os.path.join(CSRC, "calib")
CALIB_LIB_PATH = os.path.join(PKG, "libmicro_engram_calib.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 vector ops stay off: the kernels are written for scalar fp32 math
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("[micro_engram] hipcc not found: the HIP kernels cannot be built")
    return path


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    sub = "calib_" if os.path.dirname(src) == CALIB_DIR else ""
    obj = os.path.join(OBJ_DIR, sub + os.path.basename(src)[:-4] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"[micro_engram] compiling {src} failed:\n{res.stdout}\n{res.stderr}")
    return obj


def calib_sources():
    return sorted(os.path.join(CALIB_DIR, f) for f in os.listdir(CALIB_DIR) if f.endswith(".hip"))


def _link(objs, path):
    tmp = path + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"[micro_engram] linking {os.path.basename(path)} failed:\n{res.stdout}\n"
                           f"{res.stderr}")
    os.replace(tmp, path)


def build(verbose=False, jobs=None):
    """Compile every kernel source and link the library (and the benchmark's calibration
    library). Returns the library path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    calib = calib_sources()
    jobs = jobs or min(len(srcs) + len(calib), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, srcs + calib))
    _link(objs[:len(srcs)], LIB_PATH)
    _link(objs[len(srcs):], CALIB_LIB_PATH)
    if verbose:
        print(f"[micro_engram] built {LIB_PATH} from {len(srcs)} sources, "
              f"{os.path.basename(CALIB_LIB_PATH)} from {len(calib)}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
