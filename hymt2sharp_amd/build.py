"""Build the native pieces of hymt2sharp_amd in-tree.

libhymt_hip.so      C ABI (include/hymt_hip.h) + gfx950 kernels, via hipcc
libhymt_synth.so    seeded input generator (plain C), via gcc
libhymt_ceilings.so the benchmark's measured ceilings (launch gap, HBM stream
                    read, MFMA and LDS rates), via hipcc
tests/c/abi_host    a plain C host of the C ABI (tests/test_c_host.py), via gcc
_san/               ASan/UBSan builds of the host-side code (build_san.py)

Run `python -m hymt2sharp_amd.build` or call build_all().
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HIP_LIB = os.path.join(PKG, "libhymt_hip.so")
SYNTH_LIB = os.path.join(PKG, "libhymt_synth.so")
CEIL_LIB = os.path.join(PKG, "libhymt_ceilings.so")

# Sources of libhymt_hip.so and the extra compiler flags of each.
HIP_SOURCES = {
    "hymt_hip.cpp": [],
    "decode_attn.hip": [],
    "prefill_attn.hip": [],
    "kv_ops.hip": [],
    "gemv.hip": [],
    "weights.cpp": [],
    "rows.hip": [],
    "gemm.cpp": [],
    # MFMA accumulators in VGPRs: in the default AGPR form the compiler moved
    # the fp32 accumulators between registers on every k step of the GEMM
    # loop (60-124 v_accvgpr_mov_b32 per stage); o projection 31.2 -> 25.2 us
    "gemm_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "ktimer.cpp": [],
}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
BUILD_DIR = os.path.join(PKG, "_build")

# Packed fp32 VALU ops are kept off: hipcc -O3 would otherwise form
# v_pk_{add,mul,fma}_f32 from scalar float code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError("build failed: " + " ".join(cmd))
    return r.stdout


def build_hip(extra=()):
    """Compile every source to an object (in parallel), then link."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs, procs = [], []
    for src, flags in HIP_SOURCES.items():
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmd = [HIPCC, *HIP_FLAGS, *flags, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for cmd, pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            sys.stderr.write(out)
            failed.append(" ".join(cmd))
    if failed:
        raise RuntimeError("build failed: " + "; ".join(failed))
    tmp = HIP_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-L/opt/rocm/lib", "-lhipblaslt",
          "-Wl,-rpath,/opt/rocm/lib", "-o", tmp])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_ceilings():
    tmp = CEIL_LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "ceilings.hip"), "-o", tmp])
    os.replace(tmp, CEIL_LIB)
    return CEIL_LIB


def build_synth():
    tmp = SYNTH_LIB + ".tmp"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", os.path.join(CSRC, "synth.c"), "-lm",
          "-o", tmp])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


C_HOST_SRC = os.path.join(ROOT, "tests", "c", "abi_host.c")
C_HOST = os.path.join(ROOT, "tests", "c", "abi_host")


def build_c_host():
    """The plain C host of the C ABI that tests/test_c_host.py runs: gcc,
    include/hymt_hip.h, linked to libhymt_hip.so by a path relative to the
    binary (so the copy on a GPU box finds the library beside it)."""
    tmp = C_HOST + ".tmp"
    _run(["gcc", "-O2", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), C_HOST_SRC,
          "-L", PKG, "-lhymt_hip", "-Wl,-rpath,$ORIGIN/../../hymt2sharp_amd", "-o", tmp])
    os.replace(tmp, C_HOST)
    return C_HOST


def build_all():
    build_synth()
    build_ceilings()
    build_hip()
    build_c_host()
    # ASan/UBSan builds of the host-side code for the CPU tests (host only;
    # they reuse the kernel objects just built)
    from . import build_san
    build_san.build_sanitized()


if __name__ == "__main__":
    build_all()
    print(HIP_LIB)
    print(SYNTH_LIB)
