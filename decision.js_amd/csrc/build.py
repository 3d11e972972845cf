"""Builds libdj.so (the HIP kernels and the C ABI of include/dj.h) for gfx950, in-tree.

    python decision.js_amd/csrc/build.py [--jobs N]

Each .hip source is compiled by hipcc to an object in decision.js_amd/csrc/_build/, then linked into
decision.js_amd/lib/libdj.so; the Node host's N-API binding (decision.js_amd/node/dj_napi.cc) is built next to
it as dj_napi.node. No cmake: the sources are few and the flags are the ones below.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "lib", "libdj.so")
SOURCES = ["dj_runtime.hip", "dj_ops.hip", "dj_gemm.hip", "dj_attn.hip", "dj_head.hip", "dj_gdn.hip", "dj_eg2.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # packed fp32 instructions are kept out of every kernel (they have given silent wrong results on these boxes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
]


# MFMA kernels keep their accumulators in ordinary VGPRs (gfx950 allows it): with AGPRs the register allocator
# shuffled the accumulators between AGPRs on every K iteration of the GEMM loop.
PER_FILE = {"dj_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "dj_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def compile_one(src: str) -> str:
    obj = os.path.join(HERE, "_build", src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, *PER_FILE.get(src, []), "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so: harmless, filtered
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int = 4) -> str:
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    build_node_addon()
    return LIB


NODE_ADDON = os.path.join(PKG, "lib", "dj_napi.node")
NODE_INCLUDE = "/usr/include/node"


def build_node_addon() -> str:
    """The N-API binding of the C ABI for the Node host (decision.js_amd/node/), next to libdj.so: plain g++
    against the system's Node headers (N-API 8), linked to libdj.so with an $ORIGIN rpath. Skipped, with a
    note, where Node's headers are absent."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        sys.stderr.write("build.py: no Node headers at /usr/include/node: the Node binding is not built\n")
        return ""
    tmp = NODE_ADDON + ".tmp"
    cmd = ["g++", "-shared", "-fPIC", "-O2", "-std=c++17", "-Wall", "-DNODE_GYP_MODULE_NAME=dj_napi",
           "-I" + NODE_INCLUDE, "-I" + os.path.join(ROOT, "include"), os.path.join(PKG, "node", "dj_napi.cc"),
           "-L" + os.path.dirname(LIB), "-ldj", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on the Node binding:\n{r.stderr}")
    os.replace(tmp, NODE_ADDON)
    return NODE_ADDON


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    print(build(ap.parse_args().jobs))
