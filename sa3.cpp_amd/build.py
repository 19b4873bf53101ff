"""Build libsa3k.so (every HIP translation unit under csrc/, gfx950) in-tree.

Usage: python sa3.cpp_amd/build.py [-j N]
Each .hip file is compiled to an object under sa3.cpp_amd/_build/ and linked into
sa3.cpp_amd/libsa3k.so. The host-side mirror of the reference trainer headers (host/) is
header-only and is compiled by its users; its benchmark driver host/mirror_bench.cpp is built into
sa3.cpp_amd/libsa3mirror.so.
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsa3k.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    # packed-fp32 VALU forms (v_pk_add/mul/fma_f32) stay off: some of their forms have given
    # wrong results on these GPUs now and then, with no error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# translation units whose results must be bit-identical to a host float loop
NO_CONTRACT = {"adamw.hip", "quant.hip"}
# MFMA accumulators in ordinary VGPRs: the attention kernels rescale and read their accumulators
# with VALU code every key block, which with AGPR accumulators costs a copy each way
MFMA_VGPR = {"attn.hip"}


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def compile_one(src):
    obj = os.path.join(OUT_DIR, src.replace(".hip", ".o"))
    flags = list(COMMON)
    if src in NO_CONTRACT:
        flags.append("-ffp-contract=off")
    if src in MFMA_VGPR:
        flags += ["-mllvm", "-amdgpu-mfma-vgpr-form"]
    cmd = [HIPCC, *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = (r.stdout + r.stderr).strip()
    # the host pass does not know the packed-fp32 feature name; that warning is expected
    out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    return src, r.returncode, out, obj


def build(jobs=8, verbose=False):
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        results = list(ex.map(compile_one, srcs))
    failed = [r for r in results if r[1] != 0]
    for src, rc, out, _ in results:
        if out and (rc != 0 or verbose):
            print(f"--- {src}\n{out}", file=sys.stderr)
    if failed:
        raise RuntimeError("HIP compile failed: " + ", ".join(r[0] for r in failed))
    objs = [r[3] for r in results]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    build_mirror_bench()
    return LIB


MIRROR_SRC = os.path.join(HERE, "host", "mirror_bench.cpp")
MIRROR_LIB = os.path.join(HERE, "libsa3mirror.so")


def build_mirror_bench():
    """libsa3mirror.so: the host mirror's default training sequence for bench.py (host C++ only)."""
    tmp = MIRROR_LIB + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-shared", "-fPIC", "-Wall", "-Wextra", "-Werror",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "host"), MIRROR_SRC, "-o", tmp,
           "-L", HERE, "-lsa3k", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("mirror bench build failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, MIRROR_LIB)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
