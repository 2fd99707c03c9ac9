"""Build libgq.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree, and
libgq_host.so (the C++ host library over it: GGUF loading, HipBackend).

Usage: python agention-infer_amd/build.py   (or __graft_entry__.build())
Each .hip under csrc/ is compiled to an object in _build/, then linked into
agention-infer_amd/libgq.so; host/*.cpp are compiled with g++ into
agention-infer_amd/libgq_host.so.  Always recompiles (the build check must
build).
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libgq.so")
HOST_OUT = os.path.join(HERE, "libgq_host.so")
HOST_SRC = os.path.join(HERE, "host")
CXX = os.environ.get("CXX", "g++")
BUILD = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # bit-exact dequant: never fuse a*b+c unless the source says fmaf()
    "-ffp-contract=off",
    # no packed-FP32 instructions (v_pk_*_f32) in generated device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    build_host()
    if verbose:
        print(f"built {OUT}", file=sys.stderr)
    return OUT


def build_host():
    """libgq_host.so: host C++ linked against libgq.so (found next to it)."""
    srcs = sorted(os.path.join(HOST_SRC, f) for f in os.listdir(HOST_SRC) if f.endswith(".cpp"))
    tmp = HOST_OUT + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-Wall", "-Wextra", "-fPIC", "-shared", *srcs,
           f"-L{HERE}", "-lgq", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host library build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, HOST_OUT)
    return HOST_OUT


if __name__ == "__main__":
    build()
