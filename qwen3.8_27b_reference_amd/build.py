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

SOURCES = ["qk_layout.hip", "qk_gemv.hip", "qk_gemm.hip", "qk_f32.hip", "qk_noalloc.hip", "qk_abi.cpp", "qk_gguf.cpp",
           "qk_shim.cpp"]

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
    build_probe()
    build_shim_check()
    build_layout_check()
    build_sanitize_check()
    return LIB


def build_probe():
    """bench.py's plain-read ceiling (csrc/qk_probe.hip -> libqkprobe.so): a library of its own, so
    that the C ABI of include/ holds only the path."""
    src = os.path.join(CSRC, "qk_probe.hip")
    out = os.path.join(HERE, "libqkprobe.so")
    cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON, "-x", "hip", "-shared", src, "-o", out + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        print(res.stderr, file=sys.stderr)
        raise RuntimeError("build of libqkprobe.so failed")
    os.replace(out + ".tmp", out)
    return out


def build_sanitize_check():
    """The host-side ABI checks under AddressSanitizer + UndefinedBehaviorSanitizer
    (tests/sanitize_check.cpp -> tests/_bin/sanitize_check): the host sources (C ABI, GGUF reader)
    compiled by g++ with the sanitizers, linked with the kernels' objects as built above (no GPU code
    is sanitized).  Run on the CPU by tests/test_sanitize.py."""
    root = os.path.dirname(HERE)
    src = os.path.join(root, "tests", "sanitize_check.cpp")
    if not os.path.exists(src):
        return None
    out_dir = os.path.join(root, "tests", "_bin")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "sanitize_check")
    san = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined"]
    host = [os.path.join(CSRC, f) for f in ("qk_abi.cpp", "qk_gguf.cpp")]
    kernels = [os.path.join(BUILD, os.path.splitext(f)[0] + ".o") for f in SOURCES if f.endswith(".hip")]
    cmd = ["g++", "-std=c++17", "-O1", "-g", *san, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", os.path.join(root, "include"), src, *host, *kernels, "-L/opt/rocm/lib", "-lamdhip64",
           "-Wl,-rpath,/opt/rocm/lib", "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        print(res.stderr[-4000:], file=sys.stderr)
        raise RuntimeError("build of tests/_bin/sanitize_check failed")
    return out


def build_layout_check():
    """Host-only check of the T16 byte maps (tests/t16_check.cpp -> tests/_bin/t16_check)."""
    root = os.path.dirname(HERE)
    src = os.path.join(root, "tests", "t16_check.cpp")
    if not os.path.exists(src):
        return None
    out_dir = os.path.join(root, "tests", "_bin")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "t16_check")
    cmd = [HIPCC, "-O1", "-std=c++17", "-x", "hip", "--offload-arch=" + ARCH, "-I", CSRC, src, "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        print(res.stderr, file=sys.stderr)
        raise RuntimeError("build of tests/_bin/t16_check failed")
    return out


def build_shim_check():
    """The test driver of the C++ shim (tests/shim_check.cpp -> tests/_bin/shim_check), linked
    against the in-tree libqk.so with an rpath, so the GPU box runs it without installing."""
    root = os.path.dirname(HERE)
    src = os.path.join(root, "tests", "shim_check.cpp")
    if not os.path.exists(src):
        return None
    out_dir = os.path.join(root, "tests", "_bin")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "shim_check")
    cmd = [HIPCC, "-O2", "-std=c++17", "-I", os.path.join(root, "include"), src, "-L", HERE, "-lqk",
           "-Wl,-rpath,$ORIGIN/../../" + os.path.basename(HERE), "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        print(res.stderr, file=sys.stderr)
        raise RuntimeError("build of tests/_bin/shim_check failed")
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
