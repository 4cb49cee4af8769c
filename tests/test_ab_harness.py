"""The A/B timing harness (hymt2sharp_amd/ab.py): key paths into the bench
line, and a variant build that replaces one source and links the package's
other objects (CPU: hipcc cross-compiles)."""
import os
import shutil
import subprocess

import pytest

from hymt2sharp_amd import ab
from hymt2sharp_amd import build as B


def test_value_at_and_bench_line():
    doc = ab.bench_line('log line\n{"a": 1}\n{"prefill": {"roofline": {"avg_us": 28.7}}, '
                        '"config5": {"by_context": {"32768": {"frac": 0.44}}}}\n')
    assert ab.value_at(doc, "prefill.roofline.avg_us") == 28.7
    assert ab.value_at(doc, "config5.by_context.32768.frac") == 0.44
    assert ab.value_at(doc, "prefill.missing") is None
    assert ab.value_at(doc, "prefill.roofline.avg_us.deeper") is None
    with pytest.raises(RuntimeError):
        ab.bench_line("no json here")


def test_summary_medians():
    s = ab.summary({"base": {"k": [3.0, 1.0, 2.0]}, "var": {"k": [None, None]}})
    assert "median base" in s and "k=2" in s and "k=n/a" in s


@pytest.mark.skipif(not all(os.path.isfile(os.path.join(B.BUILD_DIR, os.path.splitext(s)[0] + ".o"))
                            for s in B.HIP_SOURCES), reason="package objects not built")
def test_variant_build_replaces_one_source(tmp_path):
    shutil.copy(os.path.join(B.CSRC, "rows.hip"), tmp_path / "rows.hip")
    lib = ab.build_variant(str(tmp_path))
    assert os.path.isfile(lib) and not (tmp_path / "rows.o").exists()
    syms = subprocess.run(["nm", "-D", "--defined-only", lib], stdout=subprocess.PIPE, text=True).stdout
    for name in ("hymt_create", "hymt_gemm_swiglu", "hymt_rows_swiglu_bf16", "hymt_attn_prefill"):
        assert f" {name}\n" in syms, name
    with pytest.raises(SystemExit):
        ab.build_variant(str(tmp_path / "empty_missing"))
