"""hymt_gemm_swiglu: the gate/up GEMM with SwiGLU fused into the MFMA
kernel's output (the reference's Gemm(..., swiglu: true),
VulkanBackend.cs:845-853), against the two calls it replaces --
hymt_gemm(OUT_BF16) into a [m][2 f] buffer (two calls for separate gate and
up weights), then hymt_rows_swiglu_bf16 -- bit for bit.  Those two calls are
checked against the fp64 product and the oracle's SiLU elsewhere
(test_gpu_gemm_mfma.py, test_gpu_prefill_model.py)."""
import numpy as np
import pytest

from hymt2sharp_amd import HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S

pytestmark = pytest.mark.gpu


def fused_and_composed(f, k, m, seed, separate=False):
    """(fused act or None if unsupported, composed act) for random Q4_K
    gate/up weights and a random bf16 x."""
    rng = np.random.default_rng(seed)
    xb = S.f32_to_bf16_bits(rng.standard_normal(m * k).astype(np.float32)).reshape(m, k)
    be = HipBackend(0)
    try:
        if separate:
            ws = [be.weight_upload(N.W_Q4_K, f, k, S.random_weight(seed + i, N.W_Q4_K, f, k)) for i in (1, 2)]
        else:
            ws = [be.weight_upload(N.W_Q4_K, 2 * f, k, S.random_weight(seed + 1, N.W_Q4_K, 2 * f, k))]
        for w in ws:
            be.weight_dense(w)
        dx, dgu, da, df = be.alloc(xb.nbytes), be.alloc(m * 2 * f * 2), be.alloc(m * f * 2), be.alloc(m * f * 2)
        be.upload(dx, xb)
        if separate:  # hymt_gemm writes [m][f] rows: the halves are joined on the host
            halves = []
            for w in ws:
                be.gemm(w, dx, m, da, out_bf16=True)
                be.sync()
                halves.append(be.download(np.empty((m, f), np.uint16), da))
            be.upload(dgu, np.ascontiguousarray(np.concatenate(halves, axis=1)))
        else:
            be.gemm(ws[0], dx, m, dgu, out_bf16=True)
        be.sync()
        be.rows_swiglu_bf16(dgu, m, f, da)
        be.sync()
        composed = be.download(np.empty((m, f), np.uint16), da)
        fused = None
        try:
            be.gemm_swiglu(ws[0], dx, m, df, up=ws[1] if separate else None)
            be.sync()
            fused = be.download(np.empty((m, f), np.uint16), df)
        except N.NotSupportedError:
            pass
        for p in (dx, dgu, da, df):
            be.free(p)
        for w in ws:
            be.weight_free(w)
    finally:
        be.Dispose()
    return fused, composed


@pytest.mark.parametrize("tile", ["128x128", "256x128", "128x256", "192x128", "192x256", "128x64", "128x96"])
def test_fused_tiles_equal_composed(monkeypatch, hip_available, tile):
    """Each tile (forced for the fused launch and the unfused GEMM alike;
    2 f = 768 is a multiple of every tile's width), a ragged token count."""
    monkeypatch.delenv("HYMT_HIP_GEMM", raising=False)
    monkeypatch.setenv("HYMT_HIP_GEMM_TILE", tile)
    fused, composed = fused_and_composed(384, 2048, 130, 61)
    assert fused is not None
    assert np.array_equal(fused, composed)


@pytest.mark.parametrize("f,k,m,separate", [
    (6144, 2048, 2048, False),   # the model's gate/up at a 2048-row prompt: 192 x 256 tiles
    (6144, 2048, 1531, True),    # separate gate and up weights, 192 x 128 tiles
    (6144, 2048, 300, False),
    (640, 2048, 4000, True),     # 2 f = 1280: 128 x 96 tiles (no 192-row width)
])
def test_fused_default_plan_equals_composed(monkeypatch, hip_available, f, k, m, separate):
    monkeypatch.delenv("HYMT_HIP_GEMM", raising=False)
    monkeypatch.delenv("HYMT_HIP_GEMM_TILE", raising=False)
    fused, composed = fused_and_composed(f, k, m, 7 + m, separate)
    assert fused is not None
    assert np.array_equal(fused, composed)
    # silu(g) u of random products: a spread of bf16 values, not a constant
    assert np.unique(composed).size > min(m * f // 8, 4096)


def test_fused_refused_where_bits_would_differ(monkeypatch, hip_available):
    """A short prompt, whose gate/up GEMM the plan splits over k (a different
    fp32 summation), and the library mode (hipBLASLt GEMMs): NotSupportedError
    and nothing written; the composed calls still run."""
    monkeypatch.delenv("HYMT_HIP_GEMM_TILE", raising=False)
    monkeypatch.delenv("HYMT_HIP_GEMM", raising=False)
    fused, _ = fused_and_composed(6144, 2048, 24, 5)
    assert fused is None
    fused, _ = fused_and_composed(448, 2048, 300, 5, True)   # 448 rows: hipBLASLt's GEMM
    assert fused is None
    monkeypatch.setenv("HYMT_HIP_GEMM", "library")
    fused, _ = fused_and_composed(384, 2048, 256, 6)
    assert fused is None


def test_fused_argument_errors(hip_available):
    be = HipBackend(0)
    try:
        g = be.weight_upload(N.W_Q8_0, 256, 2048, S.random_weight(1, N.W_Q8_0, 256, 2048))
        u = be.weight_upload(N.W_Q8_0, 128, 2048, S.random_weight(2, N.W_Q8_0, 128, 2048))
        dx, da = be.alloc(16 * 2048 * 2), be.alloc(16 * 256 * 2)
        with pytest.raises(N.InvalidOperationError):
            be.gemm_swiglu(g, dx, 16, da)   # no dense copy yet
        be.weight_dense(g)
        be.weight_dense(u)
        with pytest.raises(N.ArgumentError):
            be.gemm_swiglu(g, dx, 16, da, up=u)   # 256 gate rows, 128 up rows
        with pytest.raises(N.ArgumentError):
            be.gemm_swiglu(g, dx, -1, da)
        be.free(dx)
        be.free(da)
        be.weight_free(g)
        be.weight_free(u)
    finally:
        be.Dispose()


_rng = np.random.default_rng(20261203)
SWEEP = [(64 * int(_rng.integers(1, 97)), int(_rng.choice([2048, 4096])), int(_rng.integers(1, 2500)),
          bool(_rng.integers(0, 2))) for _ in range(10)]


def test_fused_random_sweep(monkeypatch, hip_available):
    """Seeded shapes (f a multiple of 64 up to 6144, k 2048 or 4096, m up to
    2500, one [gate; up] weight or two): wherever the fused launch runs it
    equals the unfused calls bit for bit; where it refuses (a k split, a width
    the MFMA GEMM does not take) the unfused calls are what the model runs."""
    monkeypatch.delenv("HYMT_HIP_GEMM", raising=False)
    monkeypatch.delenv("HYMT_HIP_GEMM_TILE", raising=False)
    ran = 0
    for i, (f, k, m, separate) in enumerate(SWEEP):
        print(f"sweep f={f} k={k} m={m} separate={separate}", flush=True)
        fused, composed = fused_and_composed(f, k, m, 900 + i, separate)
        if fused is not None:
            ran += 1
            assert np.array_equal(fused, composed), (f, k, m, separate)
    assert ran >= 3, ran
