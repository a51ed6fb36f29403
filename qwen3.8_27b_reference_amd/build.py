"""Builds libqk.so (the HIP kernels + C ABI) in-tree for gfx950 with hipcc.

Usage: python qwen3.8_27b_reference_amd/build.py [--jobs N]

Every HIP translation unit is compiled with packed-FP32 code generation disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops): hipcc would otherwise fuse float pairs into
v_pk_*_f32 instructions, which this build avoids on MI355X.  hipcc's host pass prints that it does
not know the feature; that line is harmless.
"""
import argparse
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqk.so")

SOURCES = ["qk_layout.hip", "qk_gemv.hip", "qk_gemm.hip", "qk_abi.cpp", "qk_shim.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON, *lang, "-c", path, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    return src, obj, res.returncode, err


def build(jobs=None, verbose=False):
    """Compiles every source and links libqk.so; raises RuntimeError on a compiler error."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    jobs = jobs or min(8, len(srcs))
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, obj, rc, err in ex.map(_compile, srcs):
            if err and (verbose or rc):
                print(f"[{src}]\n{err}", file=sys.stderr)
            if rc:
                raise RuntimeError(f"hipcc failed on {src}")
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        print(res.stderr, file=sys.stderr)
        raise RuntimeError("link of libqk.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
