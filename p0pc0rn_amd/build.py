"""Builds the gfx950 library, its Node N-API addon and the CPU oracle, in-tree.

    python -m p0pc0rn_amd.build            # everything
    python -m p0pc0rn_amd.build lib napi   # a subset

Outputs (git-ignored, but carried to the GPU box with the tree):
    p0pc0rn_amd/libp0pc0rn_hip.so     the C-ABI library (include/p0pc0rn.h)
    p0pc0rn_amd/js/p0pc0rn.node       the N-API addon the Node host loads
    oracle/libq4oracle.so             the CPU oracle (test infrastructure)
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libp0pc0rn_hip.so")
NAPI = os.path.join(PKG, "js", "p0pc0rn.node")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE = os.path.join(ORACLE_DIR, "libq4oracle.so")

HIP_SOURCES = ["runtime.hip", "gemv.hip", "chain_pipe.hip", "chain_wide.hip", "gemv_m01_04.hip", "gemv_m05_08.hip", "gemv_m09_12.hip",
               "gemv_m13_16.hip", "gemm.hip", "util.hip", "misc.hip", "gemv_q8.hip", "pack.hip"]
# packed-fp32 instructions are disabled on purpose: hipcc -O3 would otherwise pair fp32 ops into v_pk_*_f32
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 library)")


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "--hip-link" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build_lib(jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    objs = []

    def compile_one(src):
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        _run([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_napi():
    """The Node addon: a thin N-API layer over the C ABI, linked against the library with an $ORIGIN rpath."""
    inc = "/usr/include/node"
    if not os.path.exists(os.path.join(inc, "node_api.h")):
        raise RuntimeError("node_api.h not found under /usr/include/node")
    tmp = NAPI + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-I" + inc, "-I" + os.path.join(ROOT, "include"),
          os.path.join(CSRC, "napi.cc"), "-L" + PKG, "-lp0pc0rn_hip", "-Wl,-rpath,$ORIGIN/..", "-o", tmp])
    os.replace(tmp, NAPI)
    return NAPI


def build_oracle():
    _run(["make", "-s", "-C", ORACLE_DIR, "-B", "libq4oracle.so"])
    return ORACLE


def build_all():
    out = [build_lib(), build_oracle()]
    out.append(build_napi())
    return out


if __name__ == "__main__":
    what = sys.argv[1:] or ["lib", "oracle", "napi"]
    for w in what:
        path = {"lib": build_lib, "napi": build_napi, "oracle": build_oracle}[w]()
        print("built", os.path.relpath(path, ROOT))
