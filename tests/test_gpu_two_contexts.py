"""Two contexts on one GPU, their work interleaved on their own streams.

Everything a call needs lives in its context: the hipBLASLt handle,
workspace, scratch output and chosen algorithms of the prefill GEMMs, the
decode split partials and the K/V cache (the reference backend owns every
device buffer, IComputeBackend.cs:14-88; one caller per backend,
ChatCompletionService.cs:11).  So work of two contexts enqueued alternately,
without synchronising between them, must give each context exactly the bits
it gives alone.  (The no-allocation decode shares one static array per GPU
and is documented to race across contexts; it is not used here.)
"""
import numpy as np
import pytest

from hymt2sharp_amd import F16, HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, new_token

pytestmark = pytest.mark.gpu


def gemm_setup(be, seed, rows, cols, m):
    raw = S.random_weight(seed, N.W_Q4_K, rows, cols)
    w = be.weight_upload(N.W_Q4_K, rows, cols, raw)
    be.weight_dense(w)
    rng = np.random.default_rng(seed)
    xb = S.f32_to_bf16_bits(rng.standard_normal((m, cols)).astype(np.float32))
    dx, dy = be.alloc(xb.nbytes), be.alloc(m * rows * 4)
    be.upload(dx, xb)
    return w, dx, dy


@pytest.mark.parametrize("rows,cols,m", [(2048, 6144, 512), (12288, 2048, 300)])
def test_gemms_of_two_contexts_interleaved(hip_available, rows, cols, m):
    ctx = [HipBackend(0), HipBackend(0)]
    try:
        bufs = [gemm_setup(be, 40 + i, rows, cols, m) for i, be in enumerate(ctx)]
        alone = []
        for be, (w, dx, dy) in zip(ctx, bufs):
            be.gemm(w, dx, m, dy)  # first call of the shape: the context tunes its choice
            be.gemm(w, dx, m, dy)
            be.sync()
            alone.append(be.download(np.empty((m, rows), np.float32), dy))
        for _ in range(4):
            for be, (w, dx, dy) in zip(ctx, bufs):
                be.gemm(w, dx, m, dy)
        for be in ctx:
            be.sync()
        for be, (w, dx, dy), ref in zip(ctx, bufs, alone):
            assert np.array_equal(be.download(np.empty((m, rows), np.float32), dy), ref)
        for be, (w, dx, dy) in zip(ctx, bufs):
            be.free(dx)
            be.free(dy)
            be.weight_free(w)
    finally:
        for be in ctx:
            be.Dispose()


def test_decode_of_two_contexts_interleaved(hip_available):
    """Each context decodes 8 steps over its own 4096-row cache; the steps
    of the two are enqueued alternately with device pointers."""
    pos0, steps = 4096, 8
    ctx, dev = [], []
    try:
        for i in range(2):
            be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, pos0 + steps, F16)
            kb, vb = cache_rows(2, pos0, salt=10 + i)
            be.UploadKv(0, 0, pos0, kb, vb)
            toks = [new_token(2, 100 * i + s, "gamma") for s in range(steps)]
            d = {}
            for name, idx in (("q", 0), ("k", 1), ("v", 2)):
                arr = np.concatenate([t[idx].ravel() for t in toks]).astype(np.float32)
                d[name] = be.alloc(arr.nbytes)
                be.upload(d[name], arr)
            for name, idx in (("qnw", 3), ("knw", 4)):
                d[name] = be.alloc(D * 4)
                be.upload(d[name], np.asarray(toks[0][idx], np.float32))
            d["out"] = be.alloc(steps * HQ * D * 4)
            ctx.append(be)
            dev.append(d)

        def step(i, s):
            be, d = ctx[i], dev[i]
            be.decode_dev(0, pos0 + s, d["q"] + s * HQ * D * 4, d["k"] + s * HKV * D * 4, d["v"] + s * HKV * D * 4,
                          d["qnw"], d["knw"], d["out"] + s * HQ * D * 4)

        alone = []
        for i in range(2):  # each context alone, then its cache rows are rewritten identically below
            for s in range(steps):
                step(i, s)
            ctx[i].sync()
            alone.append(ctx[i].download(np.empty(steps * HQ * D, np.float32), dev[i]["out"]))
        for s in range(steps):
            for i in range(2):
                step(i, s)
        for be in ctx:
            be.sync()
        for i in range(2):
            got = ctx[i].download(np.empty(steps * HQ * D, np.float32), dev[i]["out"])
            assert np.array_equal(got, alone[i])
    finally:
        for be, d in zip(ctx, dev):
            for p in d.values():
                be.free(p)
        for be in ctx:
            be.Dispose()
