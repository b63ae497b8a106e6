"""Build libtabinfer.so (gfx950) from tabinfer_amd/csrc with hipcc, in-tree, and the
Node.js addon tabinfer_amd/host/tabinfer.node over it (when Node's headers are present).

    python -m tabinfer_amd.build [--force]

Every .hip file compiles to its own object under tabinfer_amd/_build/ (in
parallel), then they link into tabinfer_amd/libtabinfer.so. Flags:
  --offload-arch=gfx950   the only target
  -ffp-contract=off       expressions round once per operation as written; the
                          kernels use fmaf explicitly where a fused multiply-add
                          is wanted, which keeps the quantizers bit-exact
  -Xclang -target-feature -Xclang -packed-fp32-ops
                          no packed-FP32 instructions are generated
"""
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtabinfer.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def hipcc():
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if p and os.path.exists(p):
            return p
    raise RuntimeError("hipcc not found (ROCm is required to build libtabinfer)")


CXXFLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _compile(src, force):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    deps = [src] + glob.glob(os.path.join(CSRC, "*.h")) + [os.path.join(INCLUDE, "ti.h")]
    if not force and os.path.exists(obj) and os.path.getmtime(obj) >= max(os.path.getmtime(d) for d in deps):
        return obj
    cmd = [hipcc()] + CXXFLAGS + ["-I", INCLUDE, "-c", src, "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (os.path.basename(src), out))
    return obj


NODE_INCLUDE = "/usr/include/node"
ADDON_SRC = os.path.join(HERE, "host", "ti_node.cc")
ADDON = os.path.join(HERE, "host", "tabinfer.node")


def build_addon(force=False):
    """g++ the N-API addon (plain C ABI of libtabinfer, no HIP code) next to its JS
    modules; it finds libtabinfer.so through an $ORIGIN-relative rpath."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return None
    deps = [ADDON_SRC, os.path.join(INCLUDE, "ti.h"), LIB]
    if not force and os.path.exists(ADDON) and os.path.getmtime(ADDON) >= max(os.path.getmtime(d) for d in deps):
        return ADDON
    cxx = shutil.which("g++") or "g++"
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-DNODE_GYP_MODULE_NAME=tabinfer", "-I", NODE_INCLUDE, "-I", INCLUDE, ADDON_SRC,
           "-L", HERE, "-ltabinfer", "-Wl,-rpath,$ORIGIN/..", "-o", ADDON + ".tmp"]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("addon build failed:\n" + r.stdout)
    os.replace(ADDON + ".tmp", ADDON)
    return ADDON


def build(force=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(8, len(srcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout)
    os.replace(tmp, LIB)
    build_addon(force=True)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
