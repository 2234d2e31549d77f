"""In-tree build of libflashdp_hip.so for gfx950 (MI355X).

Each HIP source under csrc/ is compiled with hipcc to an object file, in
parallel, then linked into ``flashdp4review_amd/libflashdp_hip.so``.  The
library is what ``flashdp4review_amd._lib`` loads with ctypes; nothing is
JIT-compiled at import time.

The per-call path of the Python operators, ``_fdp_call`` (csrc/py/fdp_call.cpp,
CPython C API, host code only), is compiled with the host C++ compiler and
linked against the library.

Usage: ``python -m flashdp4review_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libflashdp_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = os.environ.get("FDP_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 instructions stay off: hipcc must not emit v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build flashdp4review_amd")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip and link the shared library; returns its path."""
    hipcc = _hipcc()
    objdir = os.path.join(PKG_DIR, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()

    def compile_one(src: str) -> str:
        obj = os.path.join(objdir, os.path.basename(src)[:-4] + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                        if "packed-fp32-ops" not in l)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{out}")
        if verbose and out.strip():
            print(out, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB_PATH)
    build_call_module()
    return LIB_PATH


CALL_SRC = os.path.join(CSRC, "py", "fdp_call.cpp")
CALL_PATH = os.path.join(PKG_DIR, "_fdp_call" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))


def build_call_module() -> str:
    """The CPython extension _fdp_call, linked against libflashdp_hip.so (rpath
    $ORIGIN, so it loads the library next to it)."""
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    tmp = CALL_PATH + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
           f"-I{sysconfig.get_paths()['include']}", CALL_SRC, "-o", tmp,
           f"-L{PKG_DIR}", "-lflashdp_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building _fdp_call failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, CALL_PATH)
    return CALL_PATH


if __name__ == "__main__":
    print(build(verbose=True))
