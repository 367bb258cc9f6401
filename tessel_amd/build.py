"""Builds tessel_amd/libtessel_hip.so: the gfx950 kernels and the C ABI of
include/tessel.h, compiled in-tree with hipcc (every source to an object in
parallel, then one shared library)."""

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtessel_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("TSL_CXX", "/opt/rocm/llvm/bin/clang++")  # host C++ with _Float16
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for every device pass: hipcc -O3 would
# otherwise form them from plain float code.
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-mf16c"]  # f16 conversions in hardware

SOURCES = ["runtime.hip", "gemm.hip", "attention.hip", "decode.hip", "rows.hip", "probe.hip"]
HOST_SOURCES = ["engine.cpp", "checkpoint.cpp"]


def _compile(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("compile failed: " + " ".join(cmd) + "\n" + err)
    return err


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    objs = []
    for s in SOURCES:
        o = os.path.join(BUILD, s.replace(".hip", ".o"))
        objs.append(o)
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
    for s in HOST_SOURCES:
        o = os.path.join(BUILD, s.replace(".cpp", ".o"))
        objs.append(o)
        jobs.append([CXX] + HOST_FLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for err in ex.map(_compile, jobs):
            if verbose and err.strip():
                print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    _compile([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


def build_sanitized():
    """tessel_amd/libtessel_hip_asan.so: the host sources (engine, checkpoint)
    built with AddressSanitizer and UndefinedBehaviorSanitizer, linked with
    the normal GPU objects (GPU sanitizers are not available on the GPU
    pool). For CPU test runs with the ASan runtime preloaded:

        LD_PRELOAD=$(clang -print-file-name=libclang_rt.asan-x86_64.so) \
        ASAN_OPTIONS=detect_leaks=0 UBSAN_OPTIONS=halt_on_error=1 \
        TSL_LIB=tessel_amd/libtessel_hip_asan.so python -m pytest tests -m "not gpu"
    """
    build()
    san = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined"]
    objs = []
    for s in HOST_SOURCES:
        o = os.path.join(BUILD, s.replace(".cpp", ".asan.o"))
        _compile([CXX] + HOST_FLAGS + san + ["-c", os.path.join(CSRC, s), "-o", o])
        objs.append(o)
    objs += [os.path.join(BUILD, s.replace(".hip", ".o")) for s in SOURCES]
    out = os.path.join(HERE, "libtessel_hip_asan.so")
    _compile([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-fsanitize=address,undefined", "-o", out] + objs)
    return out


def build_poisoned():
    """tessel_amd/libtessel_hip_poison.so: the GPU sources built with
    -DTSL_POISON_LDS (every kernel fills its LDS with NaN words before it
    starts, so a read of LDS nothing wrote shows up in the outputs), linked
    with the normal host objects. On a GPU:

        TSL_LIB=tessel_amd/libtessel_hip_poison.so python -m pytest tests -m gpu
    """
    build()
    jobs, objs = [], []
    for s in SOURCES:
        o = os.path.join(BUILD, s.replace(".hip", ".poison.o"))
        objs.append(o)
        jobs.append([HIPCC] + HIP_FLAGS + ["-DTSL_POISON_LDS", "-c", os.path.join(CSRC, s), "-o", o])
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(_compile, jobs))
    objs += [os.path.join(BUILD, s.replace(".cpp", ".o")) for s in HOST_SOURCES]
    out = os.path.join(HERE, "libtessel_hip_poison.so")
    _compile([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", out] + objs)
    return out


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(build_sanitized())
    elif "--poison" in sys.argv:
        print(build_poisoned())
    else:
        print(build(verbose=True))
