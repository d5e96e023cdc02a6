"""Build recipe for the MI355X training-path library and its bindings.

Produces, in-tree:
  forge-llm_amd/lib/libforge_hip.so   HIP kernels + the C ABI (include/forge_hip.h)
  forge-llm_amd/lib/forge_napi.node   thin N-API addon over the C ABI (JS host)

Every HIP source is compiled for gfx950 only, with packed-fp32 instruction
selection disabled (the hardware's packed fp32 forms are not used here).

Usage:  python forge-llm_amd/build.py [--jobs N]
"""
import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-I", INCLUDE,
]
NODE_INCLUDE = "/usr/include/node"

HIP_SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), r.stdout))
    return r.stdout


def _compile_hip(src):
    obj = os.path.join(OBJ, src.replace(".hip", ".o"))
    _run([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build(jobs=None):
    os.makedirs(LIB, exist_ok=True)
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile_hip, HIP_SOURCES))
    so = os.path.join(LIB, "libforge_hip.so")
    tmp = so + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, so)

    # N-API addon: plain C++ against the C ABI; node resolves napi_* at load.
    if os.path.isdir(NODE_INCLUDE) and os.path.exists(os.path.join(CSRC, "napi_addon.cpp")):
        node = os.path.join(LIB, "forge_napi.node")
        tmpn = node + ".tmp"
        _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-I", NODE_INCLUDE, "-I", INCLUDE,
              os.path.join(CSRC, "napi_addon.cpp"), "-o", tmpn, "-L", LIB, "-lforge_hip",
              "-Wl,-rpath,$ORIGIN"])
        os.replace(tmpn, node)
    return so


def clean():
    shutil.rmtree(OBJ, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    print(build(a.jobs))
    sys.exit(0)
