#!/usr/bin/env python3
"""Benchmark of HyMT2Sharp's attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the one the headline metric is quoted on):
one full 32-layer decode step, batch 1, at context 4096 -- per layer 16 q /
4 kv heads, head_dim 128, fp32 q, fp16 KV cache, RoPE at position 4096,
per-head RMSNorm on q and k -- as 32 launches of the fused decode kernel over
32 distinct layers' KV.  A step is one such 32-layer pass; inputs are resident
in HBM (device pointers) before the timed region.  Four independent KV sets
(4 x 32 layers, > 1 GiB) rotate so the 256 MiB MALL cannot serve the reads.

Also measured (secondary): causal prefill of 2048
tokens through one layer, bf16 inputs, bf16 MFMA with fp32 accumulation,
K/V written into an empty cache.

Printed: ONE JSON line.  `value` is decode-attention HBM GB/s: algorithmic
bytes per step / GPU time per step, from HIP events recorded on the
backend's stream around the whole timed region.  `roofline` prices the
dominant kernel, decode_attn: the call's algorithmic bytes over that
kernel's own mean duration, from HIP events recorded around each of its
launches on the backend's stream (a second pass over the same calls on a
context's quiet timing mode, hymt_timing_enable); `roofline.call` prices the whole
call (both launches) the same way; `traffic` is read from
profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE per call) when
present.  `decode.step_spread` / `prefill.call_spread` are the median and
p10/p90 of 200 launches timed one by one after 20 untimed ones; after them
the replayed step's first layer is compared bit for bit with an eager call
on the same inputs (`decode.replay_vs_eager`).  `prefill` carries the prefill TFLOP/s with the flash kernel's MFMA
roofline; `config1`, `config4` and `config5` are the other configurations;
`gemv` times the weight GEMVs at the decode step's shapes; `ceilings` are
rates measured on this GPU (launch gap, HBM stream read, MFMA, LDS); `model`
is the whole 32-layer hunyuan-dense model (decode tokens/s at position 4096,
prompt prefill tokens/s).  `cpu_baseline` is the C oracle (port of Ops.cs)
on this host's cores, multi-threaded and on one thread, with the host's CPU
model and ISA.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hymt2sharp_amd import BF16, F16, F32, HipBackend  # noqa: E402
from hymt2sharp_amd import synth as S  # noqa: E402
from hymt2sharp_amd import _native as N  # noqa: E402

HQ, HKV, D = 16, 4, 128
BASE, EPS = 10000.0, 1e-6
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

CTX = 4096                      # cached positions; the new token sits at 4096
LAYERS = 32
NSETS = 4                       # KV sets rotated across steps


def decode_bytes_per_layer(L, kv_bytes=2):
    """Algorithmic HBM bytes of one layer's decode: K+V rows read, q in,
    out, the appended K/V row, the two gamma vectors."""
    return 2 * L * HKV * D * kv_bytes + HQ * D * 4 * 2 + 2 * HKV * D * kv_bytes + 2 * D * 4


def prefill_flops(P0, seq):
    """Causal prefill FLOPs: 4*D*Hq*sum_i (P0 + i + 1) (QK^T and PV)."""
    return 4 * D * HQ * (seq * P0 + seq * (seq + 1) // 2)


class HipEvents:
    """hipEvent timing on the backend's own stream."""

    def __init__(self, stream):
        self.L = ctypes.CDLL("libamdhip64.so")
        self.stream = ctypes.c_void_p(stream)
        for f in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize",
                  "hipEventElapsedTime", "hipEventDestroy"):
            getattr(self.L, f).restype = ctypes.c_int

    def new(self):
        e = ctypes.c_void_p()
        assert self.L.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e):
        assert self.L.hipEventRecord(e, self.stream) == 0

    def elapsed_ms(self, a, b):
        assert self.L.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.L.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, e):
        self.L.hipEventDestroy(e)


SPREAD_LAUNCHES = 200           # per-launch spread: launches timed one by one ...
SPREAD_WARMUP = 20              # ... after this many untimed ones


def spread(ev, fn, n=SPREAD_LAUNCHES, warm=SPREAD_WARMUP):
    """Median and p10/p90 (microseconds) of `n` back-to-back launches of
    fn() after `warm` untimed ones, each bracketed by its own pair of HIP
    events on the backend's stream (the launches still run back to back: the
    events are recorded between them, not waited on until the end)."""
    for _ in range(warm):
        fn()
    evs = [(ev.new(), ev.new()) for _ in range(n)]
    for a, b in evs:
        ev.record(a)
        fn()
        ev.record(b)
    us = np.array([ev.elapsed_ms(a, b) * 1e3 for a, b in evs])
    for a, b in evs:
        ev.destroy(a)
        ev.destroy(b)
    p10, med, p90 = np.percentile(us, [10, 50, 90])
    return {"n": n, "warmup": warm, "median_us": round(float(med), 3), "p10_us": round(float(p10), 3),
            "p90_us": round(float(p90), 3), "mean_us": round(float(us.mean()), 3)}


def kernel_means(be, names):
    """{kernel: {launches, avg_us}} of the timed calls so far."""
    out = {}
    for name in names:
        try:
            n, us = be.timing(name)
        except N.ArgumentError:
            continue  # never launched (e.g. no merge for a single split)
        out[name] = {"launches": n, "avg_us": round(us / n, 3)}
    return out


def decode_pool(config, ctx, n=8):
    """`n` distinct seeded cache contents [ctx][Hkv*D] as bf16 bits."""
    scale = 1.0 / np.sqrt(D)
    return [(S.f32_to_bf16_bits(S.normal(S.seed(config, S.KCACHE, i), (ctx, HKV * D), scale)),
             S.f32_to_bf16_bits(S.normal(S.seed(config, S.VCACHE, i), (ctx, HKV * D), scale)))
            for i in range(n)]


def time_decode(config, ctx, kv_dtype, steps, warmup, layers_per_step=LAYERS, min_bytes=1 << 30,
                norm=True, graph=True, kernel_timing=False, with_spread=True):
    """Decode attention at position `ctx` (L = ctx + 1) over distinct layers.

    A step is `layers_per_step` decode calls, one per layer, in stream order
    (each call's kernels finish before the next call's start, as in the
    layer loop of a decode step).  Enough layer caches rotate across steps
    that the resident set exceeds `min_bytes`, so the 256 MiB MALL cannot
    serve the KV reads.  Inputs (q, k, v, gammas) are device-resident.
    Returns per-call and per-step times from HIP events on the backend's
    stream around the whole timed region.  norm=False passes no gamma
    vectors (the QK norm step is skipped).  kernel_timing: afterwards,
    `steps` more steps call by call with quiet per-kernel timing on
    (hymt_timing_enable: the dispatch of each kernel stamps HIP events on the
    launch stream); returns each kernel's mean duration ("kernels")."""
    L = ctx + 1
    kvb = 4 if kv_dtype == F32 else 2
    bpl = decode_bytes_per_layer(L, kvb)
    nsets = max(1, -(-min_bytes // (bpl * layers_per_step)))
    nl = layers_per_step * nsets
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS)
    be.create_cache(nl, L, kv_dtype)
    pool = decode_pool(config, ctx)
    for layer in range(nl):
        kb, vb = pool[layer % len(pool)]
        be.UploadKv(layer, 0, ctx, kb, vb)
    scale = 1.0 / np.sqrt(D)
    q = S.normal(S.seed(config, S.Q), (nl, HQ * D), scale)
    k = S.normal(S.seed(config, S.KNEW), (nl, HKV * D), scale)
    v = S.normal(S.seed(config, S.VNEW), (nl, HKV * D), scale)
    gq = S.uniform(S.seed(config, S.GQ), (nl, D), 0.9, 1.1)
    gk = S.uniform(S.seed(config, S.GK), (nl, D), 0.9, 1.1)
    dq, dk, dv = be.alloc(q.nbytes), be.alloc(k.nbytes), be.alloc(v.nbytes)
    dgq, dgk, dout = be.alloc(gq.nbytes), be.alloc(gk.nbytes), be.alloc(q.nbytes)
    for dptr, arr in ((dq, q), (dk, k), (dv, v), (dgq, gq), (dgk, gk)):
        be.upload(dptr, arr)

    def record(s):
        base_layer = (s % nsets) * layers_per_step
        for l in range(layers_per_step):
            i = base_layer + l
            be.decode_dev(i, ctx, dq + i * HQ * D * 4, dk + i * HKV * D * 4, dv + i * HKV * D * 4,
                          dgq + i * D * 4 if norm else None, dgk + i * D * 4 if norm else None,
                          dout + i * HQ * D * 4)

    ev = HipEvents(be.stream())
    for s in range(max(warmup, nsets)):  # every layer set once eagerly before recording
        record(s)
    be.sync()
    graphs = []
    if graph:
        for s in range(nsets):
            be.graph_begin()
            record(s)
            graphs.append(be.graph_end())
        step = lambda s: be.graph_launch(graphs[s % nsets])  # noqa: E731
    else:
        step = record
    for s in range(warmup):
        step(s)
    be.sync()
    # timed region: K whole steps between two events, synchronised both sides
    e0, e1 = ev.new(), ev.new()
    t0 = time.perf_counter()
    ev.record(e0)
    for s in range(steps):
        step(s)
    t_submit = time.perf_counter() - t0
    ev.record(e1)
    be.sync()
    wall = time.perf_counter() - t0
    gpu_ms = ev.elapsed_ms(e0, e1)
    ev.destroy(e0)
    ev.destroy(e1)
    # per-step spread over SPREAD_LAUNCHES steps, rotating the KV sets as above
    last = (steps - 1) % nsets
    step_spread = None
    if with_spread:
        it = iter(range(1 << 30))
        step_spread = spread(ev, lambda: step(next(it)))
        be.sync()
        last = (SPREAD_LAUNCHES + SPREAD_WARMUP - 1) % nsets
    # the last step replayed set `last`; its first layer's output must be the
    # bits an eager call on the same inputs gives (the call rewrites the same
    # cache row with the same values)
    i0 = last * layers_per_step
    replayed = np.empty(HQ * D, np.float32)
    be.download(replayed, dout + i0 * HQ * D * 4)
    dchk = be.alloc(HQ * D * 4)
    be.decode_dev(i0, ctx, dq + i0 * HQ * D * 4, dk + i0 * HKV * D * 4, dv + i0 * HKV * D * 4,
                  dgq + i0 * D * 4 if norm else None, dgk + i0 * D * 4 if norm else None, dchk)
    eager_out = np.empty(HQ * D, np.float32)
    be.download(eager_out, dchk)
    be.free(dchk)
    replay_bits_equal = bool(np.array_equal(replayed.view(np.uint32), eager_out.view(np.uint32)))
    assert replay_bits_equal, "the timed step's output differs from an eager call on the same inputs"
    for g in graphs:
        be.graph_destroy(g)
    kernels = None
    if kernel_timing:
        be.timing_enable(2)
        for s in range(steps):
            record(s)
        be.sync()
        be.timing_enable(0)
        kernels = kernel_means(be, ("decode_attn", "decode_merge"))

    out = np.empty((nl, HQ * D), np.float32)
    be.download(out, dout)
    assert np.all(np.isfinite(out))
    for p in (dq, dk, dv, dgq, dgk, dout):
        be.free(p)
    be.Dispose()

    calls = steps * layers_per_step
    call_us = gpu_ms * 1e3 / calls
    return {
        "L": L,
        "ms_per_step": gpu_ms / steps,
        "wall_ms_per_step": wall * 1e3 / steps,
        "call_us": call_us,
        "host_submit_us_per_call": t_submit * 1e6 / calls,
        "submission": "recorded step (hymt_graph_launch)" if graph else "one hymt_attn_decode per layer",
        "gbs": bpl / (call_us * 1e-6) / 1e9,
        "bytes_per_layer": bpl,
        "layers_resident": nl,
        "tokens_per_s": 1e3 / (gpu_ms / steps),
        "kernels": kernels,
        "step_spread": step_spread,
        "call_spread_us": {k: round(step_spread[k] / layers_per_step, 3)
                           for k in ("median_us", "p10_us", "p90_us")} if step_spread else None,
        "replay_vs_eager": "bit-identical" if replay_bits_equal else "differs",
    }


def time_prefill(config, p0, seq, kv_dtype, io_dtype, steps, warmup, kernel_timing=False, with_spread=True):
    """One prefill chunk of `seq` tokens at positions [p0, p0+seq) over a cache
    holding `p0` seeded positions: the chunk's K/V are appended and every row
    attends causally over [0, p0+row].  Repeating the call rewrites the same
    rows with the same values, so each timed call does identical work.
    kernel_timing: afterwards `steps` more calls with quiet per-kernel timing
    on (as in time_decode); returns each kernel's mean duration ("kernels")."""
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, p0 + seq, kv_dtype)
    if p0:
        kb, vb = decode_pool(config, p0, 1)[0]
        be.UploadKv(0, 0, p0, kb, vb)
    scale = 1.0 / np.sqrt(D)
    q = S.normal(S.seed(config, S.Q), (seq, HQ * D), scale)
    k = S.normal(S.seed(config, S.KNEW), (seq, HKV * D), scale)
    v = S.normal(S.seed(config, S.VNEW), (seq, HKV * D), scale)
    if io_dtype == BF16:
        q, k, v = map(S.f32_to_bf16_bits, (q, k, v))
    dq, dk, dv = be.alloc(q.nbytes), be.alloc(k.nbytes), be.alloc(v.nbytes)
    dout = be.alloc(seq * HQ * D * 4)
    for dptr, arr in ((dq, q), (dk, k), (dv, v)):
        be.upload(dptr, arr)
    ev = HipEvents(be.stream())

    def run():
        be.prefill_dev(0, p0, seq, dq, dk, dv, io_dtype, None, None, dout)

    for _ in range(warmup):
        run()
    be.sync()
    e0, e1 = ev.new(), ev.new()
    ev.record(e0)
    for _ in range(steps):
        run()
    ev.record(e1)
    be.sync()
    ms = ev.elapsed_ms(e0, e1) / steps
    ev.destroy(e0)
    ev.destroy(e1)
    call_spread = spread(ev, run) if with_spread else None
    be.sync()
    kernels = None
    if kernel_timing:
        be.timing_enable(2)
        for _ in range(steps):
            run()
        be.sync()
        be.timing_enable(0)
        kernels = kernel_means(be, ("prefill_kv", "prefill_flash", "prefill_merge"))
    out = np.empty((seq, HQ * D), np.float32)
    be.download(out, dout)
    assert np.all(np.isfinite(out))
    for p in (dq, dk, dv, dout):
        be.free(p)
    be.Dispose()
    fl = prefill_flops(p0, seq)
    return {"ms_per_call": ms, "tflops": fl / (ms * 1e-3) / 1e12, "flops": fl,
            "tokens_per_s": seq / (ms * 1e-3), "kernels": kernels, "call_spread": call_spread,
            "tflops_at_median": fl / (call_spread["median_us"] * 1e-6) / 1e12 if call_spread else None}


GEMV_CASES = [  # (name, weight type, rows, cols): the decode step's matrix shapes
    ("q4k_gate_up", N.W_Q4_K, 12288, 2048), ("q4k_down", N.W_Q4_K, 2048, 6144),
    ("q4k_qkv", N.W_Q4_K, 3072, 2048), ("q2c_gate_up", N.W_Q2_0C, 12288, 2048),
    ("q2c_down", N.W_Q2_0C, 2048, 6144), ("stq_gate_up", N.W_STQ1_0, 12288, 2048),
    ("q8_gate_up", N.W_Q8_0, 12288, 2048), ("q6k_lm_head", N.W_Q6_K, 120818, 2048),
]


def time_gemv(reps=200, min_bytes=320 << 20):
    """y += W x at the decode step's shapes, one call per copy of W, cycling
    over enough copies (> the 256 MB MALL) that every call streams W from HBM.
    GB/s counts the GGUF bytes of W (the algorithmic weight stream)."""
    be = HipBackend(0)
    out = {}
    try:
        ev = HipEvents(be.stream())
        for name, wt, rows, cols in GEMV_CASES:
            raw = S.random_weight(S.seed(6, 20, wt), wt, rows, cols)
            nbytes = len(raw)
            copies = max(2, -(-min_bytes // nbytes))
            ws = [be.weight_upload(wt, rows, cols, raw) for _ in range(copies)]
            x = np.ones(cols, np.float32) / cols
            dx, dy = be.alloc(cols * 4), be.alloc(rows * 4)
            be.upload(dx, x)
            be.upload(dy, np.zeros(rows, np.float32))
            n = max(reps, copies)
            for i in range(copies):
                be.gemv(ws[i], dx, dy, True)
            be.sync()
            e0, e1 = ev.new(), ev.new()
            ev.record(e0)
            for i in range(n):
                be.gemv(ws[i % copies], dx, dy, True)
            ev.record(e1)
            be.sync()
            us = ev.elapsed_ms(e0, e1) / n * 1e3
            ev.destroy(e0)
            ev.destroy(e1)
            for w in ws:
                be.weight_free(w)
            be.free(dx)
            be.free(dy)
            gbs = nbytes / (us * 1e-6) / 1e9
            out[name] = {"rows": rows, "cols": cols, "bytes": nbytes, "us": round(us, 3),
                         "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
    finally:
        be.Dispose()
    return out


GEMM_SHAPES = [  # (name, n features, k, flags): the prefill GEMMs of the model (hidden 2048, FFN 6144)
    ("qkv", 3072, 2048, "bf16"), ("o", 2048, 2048, "acc"), ("gate_up", 12288, 2048, "bf16"),
    ("down", 2048, 6144, "acc"),
]
GEMM_TILES = ["128x128", "256x128", "128x256", "192x128", "192x256", "128x64", "128x96", "128x128,2", "128x256,2",
              "128x64,2"]


def time_gemm(ms=(512, 2048), reps=10, rounds=5):
    """The prefill GEMMs y (+)= x W^T at the model's shapes: hipBLASLt's first
    heuristic choice (HYMT_HIP_GEMM=library), the hand-written MFMA kernel with
    its own tile plan (HYMT_HIP_GEMM=mfma), and the MFMA kernel with each tile forced
    (HYMT_HIP_GEMM_TILE).  HIP events around `reps` back-to-back calls on
    the backend's stream, `rounds` rounds interleaving every candidate, the
    median per candidate (one pass per candidate in turn let clock drift move
    one kernel by 10-15 % between candidates); o and down accumulate into
    fp32, q/k/v and gate/up write bf16 (as hymt_model_prefill calls them).
    For gate/up also the GEMM with its SwiGLU: hipBLASLt's or the MFMA
    plan's GEMM followed by the row kernel (hymt_rows_swiglu_bf16), and the
    fused launch (hymt_gemm_swiglu) that hymt_model_prefill runs.
    Each context reads HYMT_HIP_GEMM when its first GEMM makes its GEMM
    state, so each mode gets a context of its own."""
    out = {}
    saved = {k: os.environ.get(k) for k in ("HYMT_HIP_GEMM", "HYMT_HIP_GEMM_TILE")}
    bes = {}
    try:
        for mode in ("hipblaslt", "mfma"):
            os.environ["HYMT_HIP_GEMM"] = "mfma" if mode == "mfma" else "library"
            os.environ.pop("HYMT_HIP_GEMM_TILE", None)
            be = HipBackend(0)
            bes[mode] = be
            # the first GEMM makes the state under this mode
            w0 = be.weight_upload(N.W_Q4_K, 128, 2048, S.random_weight(1, N.W_Q4_K, 128, 2048))
            be.weight_dense(w0)
            dx, dy = be.alloc(2048 * 2), be.alloc(128 * 4)
            be.upload(dx, np.zeros(2048, np.uint16))
            be.gemm(w0, dx, 1, dy)
            be.sync()
            be.free(dx)
            be.free(dy)
            be.weight_free(w0)
        os.environ.pop("HYMT_HIP_GEMM", None)
        for name, n, k, kind in GEMM_SHAPES:
            raw = S.random_weight(S.seed(7, n, k), N.W_Q4_K, n, k)
            ws = {}
            bufs = {}
            acts = {}
            swi = name == "gate_up"
            mmax = max(ms)
            x = S.f32_to_bf16_bits(S.normal(S.seed(7, k, 1), (mmax, k), 1.0))
            for mode, be in bes.items():
                w = be.weight_upload(N.W_Q4_K, n, k, raw)
                be.weight_dense(w)
                dx = be.alloc(x.nbytes)
                dy = be.alloc(mmax * n * (2 if kind == "bf16" else 4))
                be.upload(dx, x)
                be.upload(dy, np.zeros(mmax * n * (1 if kind == "bf16" else 2), np.uint16) if kind == "bf16"
                          else np.zeros(mmax * n, np.float32))
                ws[mode] = w
                bufs[mode] = (dx, dy)
                if swi:
                    acts[mode] = be.alloc(mmax * n)  # [m][n / 2] bf16

            def run(mode, m, tile, calls, op="gemm"):
                be = bes[mode]
                if tile is None:
                    os.environ.pop("HYMT_HIP_GEMM_TILE", None)
                else:
                    os.environ["HYMT_HIP_GEMM_TILE"] = tile
                dx, dy = bufs[mode]
                ev = HipEvents(be.stream())
                gemm = lambda: be.gemm(ws[mode], dx, m, dy, accumulate=kind == "acc", out_bf16=kind == "bf16")
                if op == "gemm":
                    call = gemm
                elif op == "rows":  # the GEMM, then the SwiGLU row kernel
                    call = lambda: (gemm(), be.rows_swiglu_bf16(dy, m, n // 2, acts[mode]))
                else:  # the fused launch
                    call = lambda: be.gemm_swiglu(ws[mode], dx, m, acts[mode])
                call()
                e0, e1 = ev.new(), ev.new()
                ev.record(e0)
                for _ in range(calls):
                    call()
                ev.record(e1)
                us = ev.elapsed_ms(e0, e1) / calls * 1e3
                ev.destroy(e0)
                ev.destroy(e1)
                os.environ.pop("HYMT_HIP_GEMM_TILE", None)
                return us

            for m in ms:
                flop = 2.0 * n * k * m
                cands = [("hipblaslt", None, "gemm"), ("mfma", None, "gemm")] + \
                    [("mfma", t, "gemm") for t in GEMM_TILES]
                if swi:
                    cands += [("hipblaslt", None, "rows"), ("mfma", None, "rows")]
                    try:
                        run("mfma", m, None, 1, "fused")
                        cands.append(("mfma", None, "fused"))
                    except N.NotSupportedError:
                        pass
                for c in cands:  # warm-up: every candidate once
                    run(c[0], m, c[1], 2, c[2])
                samples = {c: [] for c in cands}
                for _ in range(rounds):  # interleaved, so clock drift weighs on all alike
                    for c in cands:
                        samples[c].append(run(c[0], m, c[1], reps, c[2]))
                med = {c: round(float(np.median(v)), 2) for c, v in samples.items()}
                rec = {"n": n, "k": k, "m": m, "out": kind, "hipblaslt_us": med[("hipblaslt", None, "gemm")],
                       "mfma_plan_us": med[("mfma", None, "gemm")],
                       "mfma_tiles_us": {t: med[("mfma", t, "gemm")] for t in GEMM_TILES}}
                if swi:
                    rec["with_swiglu_us"] = {"hipblaslt_then_rows": med[("hipblaslt", None, "rows")],
                                             "mfma_then_rows": med[("mfma", None, "rows")],
                                             "fused": med.get(("mfma", None, "fused"))}
                rec["hipblaslt_tflops"] = round(flop / (rec["hipblaslt_us"] * 1e-6) / 1e12, 1)
                rec["mfma_plan_tflops"] = round(flop / (rec["mfma_plan_us"] * 1e-6) / 1e12, 1)
                out[f"{name}_m{m}"] = rec
            for mode, be in bes.items():
                be.weight_free(ws[mode])
                for b in bufs[mode]:
                    be.free(b)
                if swi:
                    be.free(acts[mode])
    finally:
        for be in bes.values():
            be.Dispose()
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    return out


def time_model(ctx=CTX, steps=20, warmup=3, kv_dtype=F16, prompt_len=2048, prefill_reps=5,
               cpu_tokens=0):
    """Whole decode step of the 32-layer hunyuan-dense model (synthetic Q4_K
    layers, Q6_K embedding and output as in a Q4_K_M file, fp16 KV) at
    position `ctx` over a resident ctx-row cache: embedding row, per layer the
    q/k/v GEMV with RMSNorm input, decode attention, output GEMV with residual,
    gate/up GEMV with RMSNorm input, down GEMV with SwiGLU input and residual,
    then the output norm and projection.  Timed two ways: recorded (one
    hymt_graph_launch per token, HIP events) and eager (ForwardStep per
    token from Python, including the logits download).  Bytes per token: the
    GGUF bytes of every weight read (one embedding row) plus the KV reads and
    writes of the attention calls.  Then a prompt_len-token prefill through
    ForwardStep (bf16 GEMMs over dense weight copies, the flash prefill
    kernel), wall clock including the logits download."""
    from hymt2sharp_amd.model import ModelConfig
    cfg = ModelConfig(eps=EPS)
    t = S.random_model(5, cfg)
    qd, kd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    layer_shapes = [(qd + 2 * kd, cfg.hidden_size), (cfg.hidden_size, qd),
                    (2 * cfg.ffn_size, cfg.hidden_size), (cfg.hidden_size, cfg.ffn_size)]
    emb = t["token_embd.weight"]
    wbytes = sum(len(x.data) for n, x in t.items() if n != "token_embd.weight") + \
        len(emb.data) // emb.rows
    kvbytes = cfg.num_layers * decode_bytes_per_layer(ctx + 1, 4 if kv_dtype == F32 else 2)
    cpu = model_cpu = None
    if cpu_tokens:
        # the oracle's decode step (C restatement, one thread, double sums) on
        # the same weights at the same position; the cache rows are zeros,
        # which costs the same
        from oracle.model import OracleModel
        om = OracleModel(cfg, t, ctx + 1, kv_dtype)
        om.step(4242, ctx)
        t0 = time.perf_counter()
        for _ in range(cpu_tokens):
            om.step(4242, ctx)
        sec = (time.perf_counter() - t0) / cpu_tokens
        del om
        cpu = {"value": round(1.0 / sec, 4), "unit": "tokens/s", "cores": 1,
               "what": "the correctness checker's speed, not a CPU baseline",
               "sample": f"{cpu_tokens} decode steps of the same model at position {ctx} after one "
                         f"warm-up ({sec:.2f} s per token), oracle/model.py over the C "
                         f"restatement (oracle/hymt_quant.c, oracle/hymt_oracle.c)"}
        # the reference's CPU decode path restated (oracle/cpu_decode.c:
        # projections over Q8_K activations with AVX2 integer dots, the
        # reference's bf16 cache, rows over threads): the model leg's CPU
        # baseline, on min(cores, 16) threads and on one
        from oracle import oracle as OR
        from oracle.model import CpuDecodePort
        port = CpuDecodePort(cfg, t, ctx + 1, OR.BF16)
        nthr = cpu_threads()
        port.step(4242, ctx, nthr)
        reps = 10
        t0 = time.perf_counter()
        for _ in range(reps):
            port.step(4242, ctx, nthr)
        sec_n = (time.perf_counter() - t0) / reps
        t0 = time.perf_counter()
        for _ in range(2):
            port.step(4242, ctx, 1)
        sec_1 = (time.perf_counter() - t0) / 2
        del port
        model_cpu = {"value": round(1.0 / sec_n, 3), "unit": "tokens/s", "cores": nthr, "kind": "port",
                     "sample": f"{reps} decode steps at position {ctx} after one warm-up ({sec_n * 1e3:.1f} ms per "
                               f"token), oracle/cpu_decode.c: the reference's CPU decode step (Q8_K activations, "
                               f"Q4_K/Q6_K integer dots, bf16 cache), same weights",
                     "single_thread": {"value": round(1.0 / sec_1, 3), "unit": "tokens/s", "cores": 1,
                                       "sample": f"2 steps on one thread ({sec_1:.2f} s per token)"}}
    be = HipBackend(0)
    try:
        be.LoadModel(t, cfg, max_tokens=ctx + 1, kv_dtype=kv_dtype)
        del t
        pool = decode_pool(2, ctx, n=4)
        for layer in range(cfg.num_layers):
            be.UploadKv(layer, 0, ctx, *pool[layer % len(pool)])
        del pool
        m, tok = be._model, 4242
        for _ in range(warmup):
            logits = be.ForwardStep([tok], ctx)
        t0 = time.perf_counter()
        for _ in range(steps):
            logits = be.ForwardStep([tok], ctx)
        eager_ms = (time.perf_counter() - t0) * 1e3 / steps
        assert np.all(np.isfinite(logits))
        be.graph_begin()
        m.step(tok, ctx)
        g = be.graph_end()
        ev = HipEvents(be.stream())
        for _ in range(warmup):
            be.graph_launch(g)
        be.sync()
        e0, e1 = ev.new(), ev.new()
        ev.record(e0)
        for _ in range(steps):
            be.graph_launch(g)
        ev.record(e1)
        be.sync()
        ms = ev.elapsed_ms(e0, e1) / steps
        ev.destroy(e0)
        ev.destroy(e1)
        be.graph_destroy(g)
        out = np.empty(cfg.vocab_size, np.float32)
        be.download(out, m.logits)
        assert np.max(np.abs(out - logits)) <= 1e-5 * np.max(np.abs(logits)), \
            "recorded step differs from the eager one"
        # prefill of a prompt_len-token prompt at position 0 (chunks of DeviceModel.PREFILL_CHUNK
        # rows, bf16 GEMMs over the dense copies), wall clock per ForwardStep
        prompt = list(np.random.default_rng(9).integers(0, cfg.vocab_size, prompt_len))
        be.ForwardStep(prompt, 0)
        t0 = time.perf_counter()
        for _ in range(prefill_reps):
            logits = be.ForwardStep(prompt, 0)
        pf_ms = (time.perf_counter() - t0) * 1e3 / prefill_reps
        assert np.all(np.isfinite(logits))
        # a first prompt of a length not seen before (its GEMM row count falls
        # in a bucket with no chosen algorithm, which is timed once), then the
        # same prompt again
        cold_len = 1531
        cold = list(np.random.default_rng(10).integers(0, cfg.vocab_size, cold_len))
        t0 = time.perf_counter()
        be.ForwardStep(cold, 0)
        cold_ms = (time.perf_counter() - t0) * 1e3
        t0 = time.perf_counter()
        be.ForwardStep(cold, 0)
        warm_ms = (time.perf_counter() - t0) * 1e3
    finally:
        be.Dispose()
    # prefill FLOPs: 2 per weight value per row, plus causal attention per layer
    params = sum(r * c for r, c in layer_shapes) * cfg.num_layers
    pf_flops = 2.0 * prompt_len * params + cfg.num_layers * prefill_flops(0, prompt_len) + \
        2.0 * cfg.vocab_size * cfg.hidden_size
    gbs = (wbytes + kvbytes) / (ms * 1e-3) / 1e9
    return {"workload": "32-layer hunyuan-dense decode step (hidden 2048, FFN 6144, vocab 120818; "
                        "Q4_K layers, Q6_K embedding/output, synthetic weights), fp16 KV, "
                        f"position {ctx} over a {ctx}-row cache",
            "tokens_per_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
            "eager_tokens_per_s": round(1e3 / eager_ms, 1), "eager_ms_per_token": round(eager_ms, 4),
            "weight_bytes": wbytes, "kv_bytes": kvbytes, "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "submission": "recorded step (hymt_graph_launch); eager = ForwardStep from Python",
            "prefill": {"prompt_tokens": prompt_len, "ms": round(pf_ms, 3),
                        "tokens_per_s": round(prompt_len / (pf_ms * 1e-3), 1),
                        "tflops": round(pf_flops / (pf_ms * 1e-3) / 1e12, 1),
                        "frac": round(pf_flops / (pf_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                        "flops": pf_flops,
                        "timing": "wall clock per ForwardStep(prompt, 0), mean of "
                                  f"{prefill_reps}, chunks of 2048 rows",
                        "unseen_length": {"prompt_tokens": cold_len, "first_ms": round(cold_ms, 3),
                                          "again_ms": round(warm_ms, 3)}},
            # cpu_baseline is the reference's CPU path restated (Q8_K
            # activations + SIMD dots); the oracle's step is the correctness
            # checker (scalar C, double sums), reported for its speed only;
            # the reference's own published CPU figure is quoted beside them.
            "cpu_baseline": model_cpu,
            "oracle_checker_step": cpu,
            "reference_published_cpu": {
                "decode_tokens_per_s": 26.55, "prefill_tokens_per_s": 423.99, "quant": "Q4_K_M",
                "hardware": "Ryzen 7 5800X, 8 threads, AVX2", "source": "README_EN.md:132,138",
                "note": "decode of 128 tokens after a 512-token context, prefill of a 512-token prompt: "
                        "other hardware, and a shorter context than this leg's"}}


def time_block_store(layers=LAYERS, ctx=CTX, reps=20):
    """The device block store at the config-2 shape (32 layers, fp16 KV): host
    time of HarvestPrefix and RestorePrefix over a ctx-token prompt (ctx / 64
    blocks), and the GPU time of one copy-on-write (a write inside a harvested
    block: every layer's K and V page copied, then the table entry updated),
    from HIP events around `reps` of them."""
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(layers, ctx + 64, F16)
    toks = (np.arange(ctx, dtype=np.int32) * 7919) % 120000
    be.MapRange(0, ctx)
    be.sync()
    t = time.perf_counter()
    for _ in range(reps):
        be.HarvestPrefix(toks, 64)
    harvest = (time.perf_counter() - t) / reps
    be.SetCacheLen(0)
    t = time.perf_counter()
    for _ in range(reps):
        be.RestorePrefix(toks, 64)
    restore = (time.perf_counter() - t) / reps
    be.SetCacheLen(ctx)
    ev = HipEvents(be.stream())
    pos = ctx - 64 + 5  # inside the last harvested block
    be.MapRange(pos, 1)  # warm-up copy
    e0, e1 = ev.new(), ev.new()
    gpu_ms = 0.0
    for _ in range(reps):
        be.SetCacheLen(pos)
        be.RestorePrefix(toks, 64)  # back onto the harvested page
        be.sync()
        ev.record(e0)
        be.MapRange(pos, 1)  # copy-on-write
        ev.record(e1)
        gpu_ms += ev.elapsed_ms(e0, e1)
    ev.destroy(e0)
    ev.destroy(e1)
    be.Dispose()
    page_bytes = HKV * 64 * D * 2
    moved = 2 * layers * page_bytes * 2  # K and V pages of every layer, read + written
    cow_us = gpu_ms * 1e3 / reps
    return {"workload": f"{layers} layers, fp16 KV, {ctx}-token prompt ({ctx // 64} blocks)",
            "harvest_us": round(harvest * 1e6, 2), "restore_us": round(restore * 1e6, 2),
            "cow_us": round(cow_us, 3), "cow_bytes": moved, "cow_gbs": round(moved / (cow_us * 1e-6) / 1e9, 1),
            "cow_note": "GPU time of one copy-on-write: the page-copy kernel and the table update"}


def measure_ceilings():
    """Ceilings measured on this GPU (libhymt_ceilings.so, HIP events): the
    cost of a dependent launch, the time to stream the decode call's bytes
    (and a 32k-context layer's, and 1 GiB) from HBM with the decode kernel's
    access pattern, the dispatch-stamped duration of an empty kernel and of
    that stream read (the floor under the per-kernel durations reported
    here), the dense bf16 MFMA rate and the LDS read rate."""
    from hymt2sharp_amd import build as B
    L = ctypes.CDLL(B.CEIL_LIB)
    d = ctypes.c_double()
    i = ctypes.c_int()

    def ck(rc):
        if rc != 0:
            raise RuntimeError(f"libhymt_ceilings call failed: hipError {rc}")

    out = {}
    for graph, name in ((1, "graph"), (0, "eager")):
        ck(L.hc_launch_gap(graph, ctypes.byref(d)))
        out[f"launch_gap_us_{name}"] = round(d.value, 3)
    stream = {}
    for label, nbytes in (("config2_layer", decode_bytes_per_layer(CTX + 1)),
                          ("ctx32k_layer", decode_bytes_per_layer(32768)), ("1GiB", 1 << 30)):
        row = {"bytes": nbytes}
        for per in (4, 8, 16, 32):  # 16, 32, 64, 128 KiB per workgroup
            for graph, name in ((1, "graph"), (0, "eager")):
                if per != 8 and not graph:
                    continue
                ck(L.hc_stream_read(ctypes.c_size_t(nbytes), per, graph, ctypes.byref(d), ctypes.byref(i)))
                row[f"{4 * per}k_us_{name}"] = round(d.value, 3)
                row[f"{4 * per}k_gbs_{name}"] = round(nbytes / (d.value * 1e-6) / 1e9, 1)
            row[f"{4 * per}k_workgroups"] = i.value
        stream[label] = row
    out["stream_read"] = stream
    # the floor under a kernel duration as the timing mode and rocprofv3 stamp
    # it: a kernel timed by itself pays the wake of an idle queue
    disp = {}
    L.hc_dispatch_duration.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    for kind, label, nbytes in ((0, "empty", 0), (1, "stream_config2_layer", decode_bytes_per_layer(CTX + 1))):
        for iso, name in ((1, "isolated"), (0, "back_to_back")):
            ck(L.hc_dispatch_duration(kind, nbytes, iso, ctypes.byref(d)))
            disp[f"{label}_us_{name}"] = round(d.value, 3)
    out["dispatch_stamped"] = disp
    # split partials handed to a merge (4 groups x 64 workgroups streaming
    # 32 KiB each, 2 KiB partials): the split kernel alone, with a second
    # dependent merge launch, and with the last-arriving workgroup merging in
    # the same launch over device-coherent stores, ticket and loads
    L.hc_handoff.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    hand = {}
    for mode, label in ((0, "split_only"), (1, "second_launch"), (2, "in_kernel_ticket")):
        ck(L.hc_handoff(mode, ctypes.byref(d)))
        hand[f"{label}_us"] = round(d.value, 3)
    out["handoff"] = hand
    mf = {}
    for w in (1, 2, 4):
        ck(L.hc_mfma_bf16(w, ctypes.byref(d)))
        mf[f"waves_per_simd_{w}"] = round(d.value, 1)
    out["mfma_bf16_tflops"] = mf
    lds = {}
    for w in (1, 2):
        ck(L.hc_lds_read(w, ctypes.byref(d)))
        lds[f"wgs_per_cu_{w}"] = round(d.value, 2)
    out["lds_read_tbs"] = lds
    cu, clk, mclk, bus = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    ck(L.hc_device_info(ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(mclk), ctypes.byref(bus)))
    out["device"] = {"cus": cu.value, "clock_mhz": clk.value // 1000, "mem_clock_mhz": mclk.value // 1000,
                     "bus_bits": bus.value}
    out["note"] = ("per-launch times of back-to-back launches on one stream: a graph of them replayed, "
                   "or enqueued one by one; stream reads rotate over > 1 GiB of buffers; dispatch_stamped: "
                   "start-to-end event stamps of one kernel (the timing mode's and rocprofv3's kernel "
                   "duration), launched alone on a drained stream or back to back")
    return out


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_host():
    """The host the CPU legs ran on (Benchmark/Program.cs:189-211 prints the
    same: processor, thread count, SIMD support).  `isa` lists the vector
    extensions the CPU reports; the oracle itself is compiled for AVX2 + FMA +
    F16C (oracle/Makefile) and uses no wider ones."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name") and model == "unknown":
                    model = ln.split(":", 1)[1].strip()
                elif ln.startswith("flags") and not flags:
                    flags = set(ln.split(":", 1)[1].split())
    except OSError:
        pass
    want = ["avx2", "fma", "f16c", "avx512f", "avx512_bf16", "avx512_fp16", "avx512_vnni", "avx_vnni",
            "amx_tile", "amx_bf16"]
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = None
    return {"cpu_model": model, "isa": [w for w in want if w in flags], "nproc": os.cpu_count(),
            "affinity": aff, "oracle_isa": "avx2+fma+f16c, OpenMP over kv heads / query rows"}


def cpu_baseline_decode(threads, layers=LAYERS, seconds=10.0):
    """The oracle (C port of Ops.AttentionDecode and the DecodeAttention steps)
    on a sample of the same workload: `layers` layers of the 4096-context
    step, repeated for about `seconds` after one warm-up, mean per rep
    (Benchmark/Program.cs:189-211).  Returns (GB/s, s per rep, reps)."""
    from oracle import oracle as O
    L = CTX + 1
    scale = 1.0 / np.sqrt(D)
    kb = S.f32_to_bf16_bits(S.normal(S.seed(2, S.KCACHE, 0), (CTX, HKV * D), scale))
    vb = S.f32_to_bf16_bits(S.normal(S.seed(2, S.VCACHE, 0), (CTX, HKV * D), scale))
    ck = O.new_cache(L, HKV, D, O.F16)
    cv = O.new_cache(L, HKV, D, O.F16)
    ck[:CTX] = O.to_storage(S.bf16_bits_to_f32(kb), O.F16)
    cv[:CTX] = O.to_storage(S.bf16_bits_to_f32(vb), O.F16)
    q = S.normal(S.seed(2, S.Q), (HQ * D,), scale)
    k = S.normal(S.seed(2, S.KNEW), (HKV * D,), scale)
    v = S.normal(S.seed(2, S.VNEW), (HKV * D,), scale)
    g = np.full(D, 1.0, np.float32)

    def one():
        for _ in range(layers):
            O.decode_attention(q, k, v, g, g, ck, cv, O.F16, HQ, HKV, D, BASE, EPS, CTX,
                               threads=threads)

    one()
    reps = 0
    t = time.perf_counter()
    while time.perf_counter() - t < seconds:
        one()
        reps += 1
    sec = (time.perf_counter() - t) / reps
    return decode_bytes_per_layer(L) * layers / sec / 1e9, sec, reps


def cpu_baseline_prefill(threads, seq=2048, seconds=10.0):
    """The oracle's prefill (Forward's 1024-token chunks of AttentionScores ->
    SoftmaxCausal -> AttentionCombine) on config 3, repeated for about
    `seconds`.  Returns (TFLOP/s, s per run, runs)."""
    from oracle import oracle as O
    scale = 1.0 / np.sqrt(D)
    q = S.bf16_bits_to_f32(S.f32_to_bf16_bits(S.normal(S.seed(3, S.Q), (seq, HQ * D), scale)))
    k = S.bf16_bits_to_f32(S.f32_to_bf16_bits(S.normal(S.seed(3, S.KNEW), (seq, HKV * D), scale)))
    v = S.bf16_bits_to_f32(S.f32_to_bf16_bits(S.normal(S.seed(3, S.VNEW), (seq, HKV * D), scale)))
    ck = O.new_cache(seq, HKV, D, O.BF16)
    cv = O.new_cache(seq, HKV, D, O.BF16)
    runs = 0
    t = time.perf_counter()
    while time.perf_counter() - t < seconds:
        O.prefill_attention(q.reshape(seq, -1), k.reshape(seq, -1), v.reshape(seq, -1), None, None,
                            ck, cv, O.BF16, HQ, HKV, D, BASE, EPS, 0, threads=threads)
        runs += 1
    sec = (time.perf_counter() - t) / runs
    return prefill_flops(0, seq) / sec / 1e12, sec, runs


def copy_calibration(nbytes=64 << 20, reps=3):
    """Device-to-device copies of a known size: the reference point for the
    FETCH_SIZE / WRITE_SIZE counters (each copy reads and writes `nbytes`)."""
    from hymt2sharp_amd import _native as N
    be = HipBackend(0)
    src, dst = be.alloc(nbytes), be.alloc(nbytes)
    for _ in range(reps):
        N.check(be._lib.hymt_memcpy(be.handle, ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, 2))
    be.free(src)
    be.free(dst)
    be.Dispose()


def load_traffic():
    """HBM bytes per call measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (scaled by the same counters on a copy of known size), kept beside the
    profiles they come from; None when absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def r4(d):
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["decode", "prefill", "configs", "gemv", "gemm", "model", "ceilings"],
                    default=None,
                    help="run one leg: the config-2 decode step, the config-3 prefill, "
                         "the other configurations (1, 4, 5), the weight GEMVs, the prefill "
                         "GEMMs, the whole-model decode step or the measured ceilings")
    ap.add_argument("--calibrate", action="store_true",
                    help="first run 64 MiB device copies (counter calibration for profiles)")
    ap.add_argument("--no-spread", action="store_true",
                    help="skip the per-launch spread statistics (the profiled runs: rocprofv3's kernel trace "
                         "crashed in hipGraphLaunch during those 220 back-to-back replays with event records)")
    ap.add_argument("--gemm-m", default="512,2048",
                    help="prompt row counts of the gemm leg, comma-separated")
    ap.add_argument("--no-graph", action="store_true",
                    help="submit decode steps call by call instead of replaying a recorded step "
                         "(for counter collection, which times dispatches one by one)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: the attention path has no multi-GPU mode in this "
              f"build (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    if args.calibrate:
        copy_calibration()
    dec = pre = None
    extra = {}
    if args.only in (None, "decode"):
        sp = not args.no_spread
        dec = time_decode(2, CTX, F16, args.steps, args.warmup, graph=not args.no_graph,
                          kernel_timing=True, with_spread=sp)
        eager = dec if args.no_graph else time_decode(2, CTX, F16, args.steps, args.warmup,
                                                      graph=False, with_spread=sp)
    if args.only in (None, "prefill"):
        pre = time_prefill(3, 0, 2048, BF16, BF16, args.steps, args.warmup, kernel_timing=True,
                           with_spread=not args.no_spread)
    if args.only in (None, "configs"):
        c1 = time_decode(1, 512, F32, args.steps, args.warmup, norm=False, graph=not args.no_graph,
                         with_spread=not args.no_spread)
        extra["config1"] = {"workload": "decode L=513, fp32 q and KV cache, QK norm off "
                                        "(the configuration names none)",
                            "unit": "GB/s", "value": round(c1["gbs"], 1), **r4(c1)}
        c4 = time_prefill(4, 8192, 256, F16, F32, args.steps, args.warmup, kernel_timing=True,
                          with_spread=not args.no_spread)
        extra["config4"] = {"workload": "prefill chunk 256 at positions 8192..8447 over an "
                                        "8192-position fp16 cache, fp32 in",
                            "unit": "TFLOP/s", "value": round(c4["tflops"], 2), **r4(c4)}
        sweep = {}
        for ctx in (1024, 4096, 16384, 32768):
            r = time_decode(5, ctx, F16, max(4, args.steps // 4), args.warmup,
                            layers_per_step=8, graph=not args.no_graph, kernel_timing=True,
                            with_spread=not args.no_spread)
            kd = (r["kernels"] or {}).get("decode_attn")
            sweep[str(ctx)] = {"gbs": round(r["gbs"], 1), "call_us": round(r["call_us"], 3),
                               "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                               "bytes": r["bytes_per_layer"], "kernels": r["kernels"],
                               "attn_frac": round(r["bytes_per_layer"] / (kd["avg_us"] * 1e-6) / 1e9
                                                  / HBM_PEAK_GBS, 4) if kd else None}
        extra["config5"] = {"workload": "decode context sweep, fp16 KV, one layer per call",
                            "unit": "GB/s", "by_context": sweep}
        extra["block_store"] = time_block_store()
    if args.only in (None, "gemv"):
        extra["gemv"] = {"workload": "decode weight GEMV y += W x (batch 1, fp32 x/y) at the "
                                     "decode step's shapes, W streamed from HBM",
                         "unit": "GB/s of GGUF weight bytes", "cases": time_gemv()}
    if args.only in (None, "gemm"):
        extra["gemm"] = {"workload": "prefill GEMMs y (+)= x W^T at the model's shapes (bf16 operands, "
                                     "fp32 accumulation; o and down accumulate into fp32, q/k/v and "
                                     "gate/up write bf16): hipBLASLt's first heuristic choice against "
                                     "the hand-written MFMA kernel, its tile plan and each tile",
                         "unit": "us per call",
                         "shapes": time_gemm(ms=tuple(int(v) for v in args.gemm_m.split(",")))}
    if args.only in (None, "ceilings"):
        extra["ceilings"] = measure_ceilings()
    if args.only in (None, "model"):
        extra["model"] = time_model(steps=max(5, args.steps // 2), warmup=args.warmup,
                                    cpu_tokens=0 if args.no_cpu else 2)

    cpu = None
    if not args.no_cpu and dec is not None:
        th = cpu_threads()
        gbs, sec, reps = cpu_baseline_decode(th, seconds=8.0)
        gbs1, sec1, reps1 = cpu_baseline_decode(1, layers=4, seconds=6.0)
        tfl, psec, runs = cpu_baseline_prefill(th, seconds=8.0)
        tfl1, psec1, runs1 = cpu_baseline_prefill(1, seq=512, seconds=6.0)
        cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": th, "kind": "port",
               "sample": f"the 32-layer 4096-context decode step (one KV set), mean of {reps} reps "
                         f"({sec * 1e3:.1f} ms per rep, {reps * sec:.1f} s), C port of "
                         f"Ops.AttentionDecode (oracle/hymt_oracle.c), fp16 KV, {th} threads",
               "single_thread": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                                 "sample": f"4 layers of the same step, mean of {reps1} reps "
                                           f"({sec1 * 1e3:.1f} ms per rep), one thread"},
               "host": cpu_host(),
               "prefill": {"value": round(tfl, 4), "unit": "TFLOP/s", "cores": th,
                           "sample": f"the 2048-token causal prefill, mean of {runs} runs "
                                     f"({psec:.3f} s per run, {runs * psec:.1f} s), C port of "
                                     f"AttentionScores/SoftmaxCausal/AttentionCombine with "
                                     f"Forward's 1024 chunking, {th} threads",
                           "single_thread": {"value": round(tfl1, 4), "unit": "TFLOP/s", "cores": 1,
                                             "sample": f"a 512-token causal prefill, mean of {runs1} "
                                                       f"runs ({psec1:.3f} s per run), one thread"}}}

    traffic = load_traffic() or {}
    rec = {
        "metric": "decode-attn HBM GB/s (% peak) @4k ctx; prefill-attn TFLOP/s (% MFMA peak)",
        "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16-kv/fp32-math", "data": "synthetic (seeded xoshiro256**, N(0,1)/sqrt(128))",
        "config": {"workload": "config 2: 32-layer decode step, batch 1, ctx 4096 (L=4097), "
                               "16q/4kv heads, head_dim 128, fp16 KV, QK RMSNorm",
                   "global_batch": 1, "seq_len": CTX + 1, "parallelism": "none (1 GPU)"},
    }
    if dec:
        rec["value"] = round(dec["gbs"], 1)
        rec["ms_per_step"] = round(dec["ms_per_step"], 4)
        rec["decode"] = r4(dec)
        rec["decode_eager"] = {"call_us": round(eager["call_us"], 3), "gbs": round(eager["gbs"], 1),
                               "host_submit_us_per_call": round(eager["host_submit_us_per_call"], 3),
                               "submission": eager["submission"]}
        # the dominant kernel, decode_attn: the call's algorithmic bytes (every
        # K/V row it reads, q, the appended row, the gammas; the 8 KiB output
        # is written by the merge) over its own mean duration, from HIP events
        # around each launch on the backend's stream
        kd = (dec["kernels"] or {}).get("decode_attn")
        kbytes = dec["bytes_per_layer"]
        if kd:
            ach = kbytes / (kd["avg_us"] * 1e-6) / 1e9
            rec["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": round(ach / HBM_PEAK_GBS, 4),
                               "traffic": traffic.get("decode_config2"),
                               "kernel": "decode_attn_mfma_kernel<F16> (decode_attn)",
                               "algorithmic_bytes": kbytes, "avg_us": kd["avg_us"],
                               "launches_timed": kd["launches"],
                               "kernels": dec["kernels"],
                               "call": {"avg_us": round(dec["call_us"], 3),
                                        "gbs": round(dec["gbs"], 1),
                                        "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
                                        "what": "one whole decode call (both launches and the gap "
                                                "between them) in the recorded step"}}
            disp = (extra.get("ceilings") or {}).get("dispatch_stamped")
            if disp:
                # the same stamps around an empty kernel and around a kernel
                # that only streams this call's bytes: the floor of avg_us
                st = disp["stream_config2_layer_us_isolated"]
                rec["roofline"]["measurement_floor"] = {
                    "empty_kernel_us": disp["empty_us_isolated"], "stream_same_bytes_us": st,
                    "stream_over_kernel": round(st / kd["avg_us"], 3),
                    "what": "dispatch-stamped durations (the stamps avg_us uses) of an empty kernel and of a "
                            "kernel streaming the call's 8.4 MB with the decode pattern, each timed alone"}
    if pre:
        rec["prefill"] = {"workload": "config 3: causal prefill 2048 tokens, one layer, bf16 in, "
                                      "bf16 MFMA fp32 acc, empty cache",
                          "value": round(pre["tflops"], 2), "unit": "TFLOP/s",
                          "ms_per_call": round(pre["ms_per_call"], 4),
                          "call_spread": pre["call_spread"],
                          "tflops_at_median": round(pre["tflops_at_median"], 2) if pre["tflops_at_median"] else None,
                          "tokens_per_s": round(pre["tokens_per_s"], 1),
                          "call_roofline": {"bound": "mfma", "achieved": round(pre["tflops"], 2),
                                            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                            "frac": round(pre["tflops"] / BF16_PEAK_TFLOPS, 4),
                                            "traffic": traffic.get("prefill_config3"),
                                            "flops": pre["flops"]}}
        kf = (pre["kernels"] or {}).get("prefill_flash")
        if kf:
            ach = pre["flops"] / (kf["avg_us"] * 1e-6) / 1e12
            rec["prefill"]["roofline"] = {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS,
                                          "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                                          "kernel": "prefill_flash_kernel<BF16> (prefill_flash)",
                                          "flops": pre["flops"], "avg_us": kf["avg_us"],
                                          "kernels": pre["kernels"]}
    rec.update(extra)
    rec["cpu_baseline"] = cpu
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
