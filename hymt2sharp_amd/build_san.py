"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the host-side C/C++,
for the CPU test suite (tests/test_sanitized_cpu.py runs it against them).

hymt2sharp_amd/_san/libhymt_hip.so
    The C ABI with its host sources (hymt_hip.cpp with the kv_pages.hpp
    bookkeeping, weights.cpp's GGUF repack, gemm.cpp, ktimer.cpp) instrumented;
    the kernel sources are linked from the normal build's objects (their device
    code is never instrumented).
hymt2sharp_amd/_san/libhymt_oracle.so
    The CPU oracle (oracle/hymt_oracle.c, hymt_quant.c, cpu_decode.c), instrumented.
hymt2sharp_amd/_san/runtime.txt
    The sanitizer runtime to preload into the Python that loads them.

Both use ROCm's clang, so one runtime (clang's shared ASan runtime, which
carries the UBSan handlers too) serves both libraries in one process.
"""
from __future__ import annotations

import os
import subprocess

from . import build as B

SAN_DIR = os.path.join(B.PKG, "_san")
SAN_HIP_LIB = os.path.join(SAN_DIR, "libhymt_hip.so")
SAN_ORACLE_LIB = os.path.join(SAN_DIR, "libhymt_oracle.so")
SAN_RUNTIME_TXT = os.path.join(SAN_DIR, "runtime.txt")
CLANG = "/opt/rocm/llvm/bin/clang"
ORACLE_DIR = os.path.join(B.ROOT, "oracle")

# host-only instrumentation: each sanitizer flag applies to the host pass only
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-g"]
HOST_SOURCES = ["hymt_hip.cpp", "weights.cpp", "gemm.cpp", "ktimer.cpp"]


def runtime_path() -> str:
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], stdout=subprocess.PIPE,
                         text=True, check=True).stdout.strip()
    if not os.path.isfile(out):
        raise RuntimeError("clang's shared ASan runtime not found: " + out)
    return out


def build_san_hip():
    """Instrumented host sources + the normal build's kernel objects."""
    os.makedirs(SAN_DIR, exist_ok=True)
    objs, procs = [], []
    for src in B.HIP_SOURCES:
        stem = os.path.splitext(src)[0]
        if src not in HOST_SOURCES:
            obj = os.path.join(B.BUILD_DIR, stem + ".o")
            if not os.path.isfile(obj):
                raise RuntimeError("build the normal library first: missing " + obj)
            objs.append(obj)
            continue
        obj = os.path.join(SAN_DIR, stem + ".o")
        objs.append(obj)
        cmd = [B.HIPCC, *B.HIP_FLAGS, *B.HIP_SOURCES[src], *HOST_SAN, "-O1", "-c", os.path.join(B.CSRC, src),
               "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for cmd, pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            failed.append(" ".join(cmd) + "\n" + out)
    if failed:
        raise RuntimeError("sanitized build failed: " + "\n".join(failed))
    tmp = SAN_HIP_LIB + ".tmp"
    B._run([B.HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *HOST_SAN, "-Xarch_host", "-shared-libasan",
            *objs, "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib", "-o", tmp])
    os.replace(tmp, SAN_HIP_LIB)


def build_san_oracle():
    """The oracle's own flags (oracle/Makefile) plus the sanitizers."""
    os.makedirs(SAN_DIR, exist_ok=True)
    tmp = SAN_ORACLE_LIB + ".tmp"
    omp = "/opt/rocm/llvm/lib"
    B._run([CLANG, "-O1", "-g", "-fPIC", "-std=c11", "-mavx2", "-mfma", "-mf16c", "-ffp-contract=off", "-fopenmp",
            "-Wall", "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
            "-shared-libasan", "-shared", os.path.join(ORACLE_DIR, "hymt_oracle.c"),
            os.path.join(ORACLE_DIR, "hymt_quant.c"), os.path.join(ORACLE_DIR, "cpu_decode.c"), "-lm", "-L" + omp, "-Wl,-rpath," + omp, "-o", tmp])
    os.replace(tmp, SAN_ORACLE_LIB)


def build_sanitized():
    build_san_oracle()
    build_san_hip()
    with open(SAN_RUNTIME_TXT, "w") as f:
        f.write(runtime_path() + "\n")


if __name__ == "__main__":
    build_sanitized()
    print(SAN_HIP_LIB)
    print(SAN_ORACLE_LIB)
