"""Properties of the gfx950 device code that no result comparison shows,
checked on the assembly hipcc emits for each HIP source with the build's own
flags (hymt2sharp_amd/build.py HIP_FLAGS):

* m0: the LDS DMA helper (lds_dma16, device_common.hpp) writes m0 in inline
  assembly and declares it clobbered, but m0 is a reserved register that the
  compiler need not save around an asm statement.  That is safe only while
  the compiler itself keeps nothing in m0, so every m0 in the kernels must be
  the helper's own `s_mov_b32 m0, sN` directly followed by its
  `global_load_lds_dwordx4`;
* packed fp32: the build disables the packed-fp32-ops feature, so no
  v_pk_{add,mul,fma}_f32 may appear (without the flag hipcc -O3 emits
  hundreds to thousands of them per source: rows.hip 340, gemv.hip 12079).
"""
import os
import re
import shutil
import subprocess

import pytest

from hymt2sharp_amd import build as B

HIPCC = B.HIPCC
SOURCES = [s for s in B.HIP_SOURCES if s.endswith(".hip")]


def _asm(tmp_path):
    procs = {}
    for src in SOURCES:
        out = tmp_path / (src + ".s")
        cmd = [HIPCC, *[f for f in B.HIP_FLAGS if f != "-fPIC"], "-Wno-inline-asm", "--cuda-device-only", "-S",
               "-I", B.CSRC, os.path.join(B.CSRC, src), "-o", str(out)]
        procs[src] = (out, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
    res = {}
    for src, (out, p) in procs.items():
        log, _ = p.communicate()
        assert p.returncode == 0, log[-2000:]
        res[src] = [ln.strip() for ln in out.read_text().splitlines()]
    return res


def _instructions(lines):
    return [ln for ln in lines if ln and not ln.startswith((";", ".")) and not ln.endswith(":")]


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not (os.path.exists(HIPCC) or shutil.which(HIPCC)):
        pytest.skip("hipcc not available")
    if os.environ.get("HYMT_SANITIZED_CHILD") == "1":
        # the sanitized rerun of the CPU suite preloads the ASan runtime,
        # which the compiler would inherit; the code checked here is the same
        pytest.skip("compiler checks run in the plain CPU suite")
    return _asm(tmp_path_factory.mktemp("asm"))


def test_m0_only_feeds_the_lds_dma(asm):
    used = 0
    for src, lines in asm.items():
        ins = _instructions(lines)
        for i, ln in enumerate(ins):
            if re.search(r"\bm0\b", ln):
                assert ln.startswith("s_mov_b32 m0, s") and ins[i + 1].startswith("global_load_lds_dwordx4"), \
                    (src, ln, ins[i + 1])
                used += 1
    assert used > 0  # the prefill flash kernel and the MFMA GEMM do use it


def test_no_packed_fp32(asm):
    for src, lines in asm.items():
        hits = [ln for ln in _instructions(lines) if re.match(r"v_pk_(add|mul|fma)_f32\b", ln)]
        assert not hits, (src, hits[:3])
