"""Build libmllm.so (HIP, gfx950) and the Node N-API addon in-tree.

    python microllm-lab_amd/build.py            # everything
    python microllm-lab_amd/build.py lib        # libmllm.so only
    python microllm-lab_amd/build.py convert    # the PGW1 converter (host C++)
    python microllm-lab_amd/build.py probe      # libmllm_probe.so: the stage probe build (stage_probe.py)

hipcc cross-compiles for gfx950 without a GPU.  All HIP code is built with
packed-FP32 instructions disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops) and without FMA contraction (the kernels spell their FMAs
out), so results do not depend on the compiler's contraction choices.

Every kernel's register and scratch usage is recorded from the compiler's
resource-usage remarks into _build/resource_usage.json, and the build fails
if any kernel uses scratch memory: a register array that the compiler moved
to scratch turns each access into a memory round trip (and adds HBM traffic).
"""
from __future__ import annotations

import json
import os
import re
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
CONVERT_SRC = os.path.join(PKG, "convert", "pgw_convert.cc")
CONVERT_LIB = os.path.join(PKG, "convert", "libpgwconvert.so")
CONVERT_BIN = os.path.join(PKG, "convert", "pgw_convert")
NAPI_OUT = os.path.join(PKG, "js", "mllm_napi.node")

HIP_SOURCES = ["mllm_ops.hip", "mllm_engine.hip", "mllm_prefill.hip", "mllm_generic.hip"]
# per-source flags: the prefill kernels consume their matrix-core results in
# VALU epilogues, so the results go to VGPRs (no AGPR-to-VGPR copies)
EXTRA_FLAGS = {"mllm_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MLLM_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-value",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


RESOURCE_JSON = os.path.join(BUILD, "resource_usage.json")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; drop that line
    lines = [ln for ln in r.stdout.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + "\n".join(lines[-60:]))
    return lines


def _resource_usage(lines):
    """{kernel: {field: value}} from -Rpass-analysis=kernel-resource-usage remarks."""
    out, cur = {}, None
    for ln in lines:
        m = re.search(r"remark: Function Name: (\S+)", ln)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\d+) \[-Rpass", ln)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    return out


PROBE_LIB = os.path.join(PKG, "libmllm_probe.so")


def build_lib(verbose: bool = False, defines=(), out: str = LIB) -> str:
    """libmllm.so, or with defines another build of the same sources (its
    objects under _build/<name>/, no resource record)."""
    objdir = BUILD if out == LIB else os.path.join(BUILD, os.path.basename(out).replace(".so", ""))
    os.makedirs(objdir, exist_ok=True)
    objs = []
    dflags = [f"-D{d}" for d in defines]

    def compile_one(src):
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        lines = _run([HIPCC, *HIP_FLAGS, *dflags, *EXTRA_FLAGS.get(src, []), "-Rpass-analysis=kernel-resource-usage",
                      "-c", os.path.join(CSRC, src), "-o", obj])
        return obj, _resource_usage(lines)

    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        results = list(ex.map(compile_one, HIP_SOURCES))
    objs = [o for o, _ in results]
    usage = {}
    for _, u in results:
        usage.update(u)
    if out == LIB:
        with open(RESOURCE_JSON, "w") as f:
            json.dump(usage, f, indent=1, sort_keys=True)
    spilled = {k: v for k, v in usage.items() if v.get("ScratchSize", 0) > 0}
    if spilled:
        raise RuntimeError("kernels use scratch memory: " + ", ".join(f"{k} ({v['ScratchSize']} B/lane)"
                                                                      for k, v in sorted(spilled.items())))
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


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


def build_convert(verbose: bool = False) -> str:
    """The PGW1 converter (host C++): libpgwconvert.so and the pgw_convert command."""
    cxx = shutil.which("g++") or "g++"
    flags = ["-O2", "-std=c++17", "-Wall", "-Wextra", f"-I{INCLUDE}"]
    tmp = CONVERT_LIB + ".tmp"
    _run([cxx, *flags, "-shared", "-fPIC", CONVERT_SRC, "-o", tmp])
    os.replace(tmp, CONVERT_LIB)
    tmp = CONVERT_BIN + ".tmp"
    _run([cxx, *flags, "-DPGW_CONVERT_MAIN", CONVERT_SRC, "-o", tmp])
    os.replace(tmp, CONVERT_BIN)
    if verbose:
        print(f"built {CONVERT_LIB} and {CONVERT_BIN}")
    return CONVERT_LIB


def build_all(verbose: bool = False):
    build_lib(verbose)
    build_napi(verbose)
    build_convert(verbose)


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what == "lib":
        build_lib(True)
    elif what == "napi":
        build_napi(True)
    elif what == "convert":
        build_convert(True)
    elif what == "probe":
        build_lib(True, defines=["MLLM_STAGE_PROBE"], out=PROBE_LIB)
    else:
        build_all(True)
