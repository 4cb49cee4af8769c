"""The hand-written prefill GEMM (hymt2sharp_amd/csrc/gemm_mfma.hip) through
hymt_gemm, forced with HYMT_HIP_GEMM=mfma, against the fp64 product of the
same bf16 operands; and the timed choice between it and hipBLASLt.

Bounds as for the library path: fp32 results within 1e-5 of sum |x w| (fp32
accumulation over k <= 6144 against double), bf16 results within one bf16
rounding of the product plus that."""
import numpy as np
import pytest

from hymt2sharp_amd import HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bf16_bits(a):
    return S.f32_to_bf16_bits(np.ascontiguousarray(a, dtype=np.float32)).reshape(np.shape(a))


def bf16_val(b):
    return S.bf16_bits_to_f32(np.ascontiguousarray(b)).reshape(np.shape(b))


def run_case(rows, cols, m, seed, kernel_names):
    """(results, kernel launch counts) of fp32 / accumulate / bf16-out GEMMs
    over a Q4_K matrix's dense copy, and the fp64 reference."""
    raw = S.random_weight(seed, N.W_Q4_K, rows, cols)
    wd = bf16_val(bf16_bits(O.dequant(N.W_Q4_K, raw, rows, cols))).astype(np.float64)
    rng = np.random.default_rng(seed)
    xb = bf16_bits(rng.standard_normal((m, cols)).astype(np.float32))
    x = bf16_val(xb).astype(np.float64)
    y0 = rng.standard_normal((m, rows)).astype(np.float32)
    be = HipBackend(0)
    try:
        be.timing_enable(2)
        w = be.weight_upload(N.W_Q4_K, rows, cols, raw)
        be.weight_dense(w)
        dx, dy, dy16 = be.alloc(xb.nbytes), be.alloc(y0.nbytes), be.alloc(m * rows * 2)
        be.upload(dx, xb)
        out = {}
        be.gemm(w, dx, m, dy)
        be.sync()
        out["f32"] = be.download(np.empty((m, rows), np.float32), dy)
        be.upload(dy, y0)
        be.gemm(w, dx, m, dy, accumulate=True)
        be.sync()
        out["acc"] = be.download(np.empty((m, rows), np.float32), dy)
        be.gemm(w, dx, m, dy16, out_bf16=True)
        be.sync()
        out["bf16"] = bf16_val(be.download(np.empty((m, rows), np.uint16), dy16)).astype(np.float64)
        counts = {}
        for k in kernel_names:
            try:
                counts[k] = be.timing(k)[0]
            except N.ArgumentError:
                counts[k] = 0
        for p in (dx, dy, dy16):
            be.free(p)
        be.weight_free(w)
    finally:
        be.Dispose()
    return out, counts, x @ wd.T, np.abs(x) @ np.abs(wd).T, y0


def check(out, ref, mag, y0):
    assert np.all(np.abs(out["f32"] - ref) <= 1e-5 * mag + 1e-6), np.max(np.abs(out["f32"] - ref) / (mag + 1e-6))
    assert np.all(np.abs(out["acc"] - (ref + y0)) <= 1e-5 * (mag + np.abs(y0)) + 1e-6)
    assert np.all(np.abs(out["bf16"] - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-5 * mag + 1e-6)


MFMA = ["gemm_mfma_out_f32", "gemm_mfma_out_bf16"]


@pytest.mark.parametrize("rows,cols,m", [
    (128, 2048, 1),      # one tile, one token
    (256, 2048, 5),
    (640, 2048, 130),    # ragged token tile
    (384, 6144, 257),    # the down projection's k; three token tiles
    (2048, 2048, 512),   # the o projection: 64 tiles, XCD-grouped order
])
def test_mfma_gemm_forced(monkeypatch, hip_available, rows, cols, m):
    monkeypatch.setenv("HYMT_HIP_GEMM", "mfma")
    out, counts, ref, mag, y0 = run_case(rows, cols, m, 1000 + rows + m, MFMA)
    check(out, ref, mag, y0)
    assert counts == {"gemm_mfma_out_f32": 2, "gemm_mfma_out_bf16": 1}


@pytest.mark.parametrize("tile", ["128x128", "256x128", "128x256", "192x128", "192x256", "128x64", "128x96"])
@pytest.mark.parametrize("split", [1, 2])
@pytest.mark.parametrize("cols,m", [(2048, 130), (6144, 257)])
def test_mfma_gemm_tiles(monkeypatch, hip_available, tile, split, cols, m):
    """Every workgroup tile, with and without the k split, on a width every
    tile divides (768 = 3 x 256 = 4 x 192) and ragged token counts; a split
    call gives the same bits on a second run (its halves meet in one
    commutative addition)."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "mfma")
    monkeypatch.setenv("HYMT_HIP_GEMM_TILE", tile + (",2" if split == 2 else ""))
    out, counts, ref, mag, y0 = run_case(768, cols, m, 3000 + m + split, MFMA)
    check(out, ref, mag, y0)
    assert counts == {"gemm_mfma_out_f32": 2, "gemm_mfma_out_bf16": 1}
    if split == 2:
        again, _, _, _, _ = run_case(768, cols, m, 3000 + m + split, MFMA)
        for key in out:
            assert np.array_equal(out[key], again[key]), key


def test_mfma_gemm_default_plans(monkeypatch, hip_available):
    """The shape rules' own choices at the model's shapes on a 512-row
    prompt (128 x 64 for q/k/v, 128 x 64 split for o and down, 192 x 128 on
    8 waves for gate/up), against the fp64 product."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "mfma")
    monkeypatch.delenv("HYMT_HIP_GEMM_TILE", raising=False)
    for rows, cols in [(3072, 2048), (12288, 2048), (2048, 2048), (2048, 6144)]:
        out, counts, ref, mag, y0 = run_case(rows, cols, 512, 4000 + rows + cols, MFMA)
        check(out, ref, mag, y0)
        assert counts == {"gemm_mfma_out_f32": 2, "gemm_mfma_out_bf16": 1}


def test_mfma_gemm_runs_and_falls_back(monkeypatch, hip_available):
    """Forced, the MFMA kernel serves every call its shape rules allow (the
    128-row range); a width that is not a multiple of 128 goes to hipBLASLt."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "mfma")
    raw = S.random_weight(5, N.W_Q4_K, 200, 2048)
    be = HipBackend(0)
    try:
        be.timing_enable(2)
        w = be.weight_upload(N.W_Q4_K, 200, 2048, raw)
        be.weight_dense(w)
        dx, dy = be.alloc(3 * 2048 * 2), be.alloc(3 * 200 * 4)
        be.upload(dx, np.zeros(3 * 2048, np.uint16))
        be.gemm(w, dx, 3, dy)                      # 200 rows: library
        be.gemm(w, dx, 3, dy, row0=0, nrows=128)   # 128 rows: MFMA kernel
        be.sync()
        assert be.timing("gemm_mfma_out_f32")[0] == 1
        assert be.timing("gemm_bf16_out_f32")[0] == 1
        be.free(dx)
        be.free(dy)
        be.weight_free(w)
    finally:
        be.Dispose()


def test_auto_choice_is_correct(monkeypatch, hip_available):
    """HYMT_HIP_GEMM=auto: the first call of a shape times the MFMA kernel
    against hipBLASLt's candidates; whichever wins, the results hold the bound."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "auto")
    out, _, ref, mag, y0 = run_case(1024, 2048, 300, 77, MFMA)
    check(out, ref, mag, y0)


@pytest.mark.parametrize("rows,cols,m,mfma", [
    (2048, 2048, 2048, True),    # o at a 2048-row prompt: the MFMA kernel
    (1024, 6144, 300, True),
    (8192, 2048, 1024, True),    # a 32 MiB weight over 1024 rows
    (200, 2048, 64, False),      # a width the MFMA kernel does not take: hipBLASLt's first choice
])
def test_default_choice_is_reproducible(monkeypatch, hip_available, rows, cols, m, mfma):
    """Unset HYMT_HIP_GEMM: the MFMA kernel wherever it fits, hipBLASLt's
    first heuristic choice elsewhere; no timing either way, so two contexts
    (each choosing on its own) give the same bits for the same inputs, and the
    results hold the bound."""
    monkeypatch.delenv("HYMT_HIP_GEMM", raising=False)
    monkeypatch.delenv("HYMT_HIP_GEMM_TILE", raising=False)
    a, counts, ref, mag, y0 = run_case(rows, cols, m, 91, MFMA)
    b, _, _, _, _ = run_case(rows, cols, m, 91, MFMA)
    check(a, ref, mag, y0)
    if mfma:
        assert counts == {"gemm_mfma_out_f32": 2, "gemm_mfma_out_bf16": 1}
    else:
        assert not any(counts.values()), counts
    for key in a:
        assert np.array_equal(a[key], b[key]), key


def test_unsplit_tiles_agree_bitwise(monkeypatch, hip_available):
    """Every unsplit tile gives the same bits (each output's k order is the
    same 32-k MFMA chain): what lets the fused gate/up + SwiGLU launch use its
    own tile and still equal the unfused calls."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "mfma")
    base = None
    for tile in ["128x128", "256x128", "128x256", "192x128", "192x256", "128x64", "128x96"]:
        monkeypatch.setenv("HYMT_HIP_GEMM_TILE", tile)
        out, _, _, _, _ = run_case(768, 2048, 130, 5150, MFMA)
        if base is None:
            base = out
        for key in out:
            assert np.array_equal(out[key], base[key]), (tile, key)


def test_library_choice_is_reproducible(monkeypatch, hip_available):
    """HYMT_HIP_GEMM=library: hipBLASLt's first heuristic choice for every
    shape, never the MFMA kernel, the same bits in two contexts."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "library")
    a, counts, ref, mag, y0 = run_case(2048, 2048, 2048, 91, MFMA)
    b, _, _, _, _ = run_case(2048, 2048, 2048, 91, MFMA)
    check(a, ref, mag, y0)
    assert not any(counts.values()), counts
    for key in a:
        assert np.array_equal(a[key], b[key]), key



def test_planned_split_runs_split_in_a_fresh_context(monkeypatch, hip_available):
    """The plan's k split of 128 x 64 tiles (the o projection on a 512-row
    prompt) runs split on a context's first call: the split workspace holds a
    ticket per tile of the plan's own tile (it was once sized for 128 x 128
    tiles, and a call whose tiles outnumbered its tickets fell back to the
    unsplit kernel, so the bits depended on which calls came before).  Each
    case is a fresh context: the plan's bits equal the forced split's and
    differ from the unsplit kernel's (a different fp32 summation order)."""
    monkeypatch.setenv("HYMT_HIP_GEMM", "mfma")
    monkeypatch.delenv("HYMT_HIP_GEMM_TILE", raising=False)
    plan, _, ref, mag, y0 = run_case(2048, 2048, 512, 55, MFMA)
    check(plan, ref, mag, y0)
    monkeypatch.setenv("HYMT_HIP_GEMM_TILE", "128x64,2")
    split, _, _, _, _ = run_case(2048, 2048, 512, 55, MFMA)
    monkeypatch.setenv("HYMT_HIP_GEMM_TILE", "128x64")
    whole, _, _, _, _ = run_case(2048, 2048, 512, 55, MFMA)
    for key in plan:
        assert np.array_equal(plan[key], split[key]), key
    assert not np.array_equal(plan["f32"], whole["f32"])
