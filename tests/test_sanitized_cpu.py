"""The CPU test suite again, in a child Python, against AddressSanitizer +
UndefinedBehaviorSanitizer builds of the host-side C/C++ (hymt2sharp_amd/
build_san.py): the C ABI's argument checks and the kv_pages.hpp page and
block-store bookkeeping on host-only contexts, the GGUF repack, and the CPU
oracle.  Any sanitizer report aborts the child (halt_on_error, no recovery),
so the child's suite must pass whole.  Leak checking is off: the Python
interpreter itself holds allocations until exit."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "hymt2sharp_amd", "_san")
CHILD = "HYMT_SANITIZED_CHILD"


@pytest.mark.skipif(os.environ.get(CHILD) == "1", reason="already the sanitized child")
def test_cpu_suite_under_asan_and_ubsan():
    hip = os.path.join(SAN, "libhymt_hip.so")
    orc = os.path.join(SAN, "libhymt_oracle.so")
    rt_txt = os.path.join(SAN, "runtime.txt")
    if not all(os.path.isfile(p) for p in (hip, orc, rt_txt)):
        pytest.skip("sanitized libraries not built (build() builds them: hymt2sharp_amd/build_san.py)")
    runtime = open(rt_txt).read().strip()
    if not os.path.isfile(runtime):
        pytest.skip("the sanitizer runtime is not installed here: " + runtime)
    env = dict(os.environ)
    env.update({
        CHILD: "1",
        "LD_PRELOAD": runtime,
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1:detect_odr_violation=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "HYMT_HIP_LIB": hip,
        "HYMT_ORACLE_LIB": orc,
        "OMP_NUM_THREADS": "4",
    })
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-q", "-x", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=900)
    out = r.stdout
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    assert r.returncode == 0, out[-6000:]
    # the child really loaded the instrumented builds
    assert " passed" in out, out[-2000:]
