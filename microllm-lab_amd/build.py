"""Build libmllm.so (HIP, gfx950) and the Node N-API addon in-tree.

    python microllm-lab_amd/build.py            # everything
    python microllm-lab_amd/build.py lib        # libmllm.so only

hipcc cross-compiles for gfx950 without a GPU.  All HIP code is built with
packed-FP32 instructions disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops) and without FMA contraction (the kernels spell their FMAs
out), so results do not depend on the compiler's contraction choices.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libmllm.so")
NAPI_SRC = os.path.join(PKG, "js", "napi", "mllm_napi.cc")
NAPI_OUT = os.path.join(PKG, "js", "mllm_napi.node")

HIP_SOURCES = ["mllm_ops.hip", "mllm_engine.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MLLM_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-value",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; drop that line
    lines = [ln for ln in r.stdout.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + "\n".join(lines[-60:]))
    return lines


def build_lib(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs = []

    def compile_one(src):
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_napi(verbose: bool = False) -> str:
    """The N-API addon links libmllm.so with an $ORIGIN-relative rpath."""
    if not os.path.exists(NAPI_SRC):
        return ""
    node_inc = "/usr/include/node"
    if not os.path.exists(os.path.join(node_inc, "node_api.h")):
        raise RuntimeError("node_api.h not found; cannot build the N-API addon")
    cxx = shutil.which("g++") or "g++"
    tmp = NAPI_OUT + ".tmp"
    _run([cxx, "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{node_inc}", f"-I{INCLUDE}", NAPI_SRC, "-o", tmp,
          f"-L{PKG}", "-l:libmllm.so", "-Wl,-rpath,$ORIGIN/.."])
    os.replace(tmp, NAPI_OUT)
    if verbose:
        print(f"built {NAPI_OUT}")
    return NAPI_OUT


def build_all(verbose: bool = False):
    build_lib(verbose)
    build_napi(verbose)


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what == "lib":
        build_lib(True)
    elif what == "napi":
        build_napi(True)
    else:
        build_all(True)
