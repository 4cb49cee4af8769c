"""Recorded call sequences (hymt_graph_*) on the GPU: a recorded decode step
and a recorded prefill replay to the same bits as the eager calls, replays
interleaved with eager work stay correct, and calls that cannot be recorded
are refused with the recording discarded.

The recorded form is what a HipBackend.ForwardStep would submit per token,
as the Vulkan backend records its decode command buffer once and replays it
(VulkanBackend.cs:326, :400-568, :677)."""
import ctypes

import numpy as np
import pytest

from hymt2sharp_amd import BF16, F16, F32, HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, new_token

pytestmark = pytest.mark.gpu


def backend(layers, cap, dtype):
    return HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(layers, cap, dtype)


def dev_inputs(be, arrays):
    ptrs = []
    for a in arrays:
        p = be.alloc(max(a.nbytes, 16))
        be.upload(p, a)
        ptrs.append(p)
    return ptrs


@pytest.mark.parametrize("pos", [700, 20480])
def test_recorded_decode_step_replays_exactly(hip_available, pos):
    """700: page ids in the kernel arguments; 20480: page ids from the
    device table, splits taking their pages in runs."""
    layers = 3
    be = backend(layers, pos + 1, F16)
    try:
        kb, vb = cache_rows(11, pos)
        for l in range(layers):
            be.UploadKv(l, 0, pos, kb, vb)
        q, k, v, qnw, knw = new_token(11, 0, "gamma", seq=layers)
        dq, dk, dv, dqn, dkn = dev_inputs(be, [q, k, v, qnw, knw])
        dout = be.alloc(q.nbytes)
        qs, ks = HQ * D * 4, HKV * D * 4

        def step():
            for l in range(layers):
                be.decode_dev(l, pos, dq + l * qs, dk + l * ks, dv + l * ks, dqn, dkn, dout + l * qs)

        step()  # eager warm-up
        eager = be.download(np.empty((layers, HQ * D), np.float32), dout)
        be.graph_begin()
        step()
        g = be.graph_end()
        try:
            for rep in range(3):
                be.upload(dout, np.zeros_like(q))  # eager work between replays
                be.graph_launch(g)
                be.sync()
                got = be.download(np.empty((layers, HQ * D), np.float32), dout)
                assert np.array_equal(got, eager), rep
        finally:
            be.graph_destroy(g)
        for p in (dq, dk, dv, dqn, dkn, dout):
            be.free(p)
    finally:
        be.Dispose()


def test_recorded_prefill_replays_exactly(hip_available):
    pos, seq = 130, 96
    be = backend(1, pos + seq, BF16)
    try:
        kb, vb = cache_rows(12, pos)
        be.UploadKv(0, 0, pos, kb, vb)
        q, k, v, qnw, knw = new_token(12, 0, "gamma", seq=seq)
        qb, kb16, vb16 = (S.f32_to_bf16_bits(x) for x in (q, k, v))
        dq, dk, dv, dqn, dkn = dev_inputs(be, [qb, kb16, vb16, qnw, knw])
        dout = be.alloc(q.nbytes)
        be.prefill_dev(0, pos, seq, dq, dk, dv, BF16, dqn, dkn, dout)
        eager = be.download(np.empty((seq, HQ * D), np.float32), dout)
        be.graph_begin()
        be.prefill_dev(0, pos, seq, dq, dk, dv, BF16, dqn, dkn, dout)
        g = be.graph_end()
        try:
            for rep in range(3):
                be.upload(dout, np.zeros_like(q))
                be.graph_launch(g)
                be.sync()
                got = be.download(np.empty((seq, HQ * D), np.float32), dout)
                assert np.array_equal(got, eager), rep
        finally:
            be.graph_destroy(g)
        for p in (dq, dk, dv, dqn, dkn, dout):
            be.free(p)
    finally:
        be.Dispose()


def test_unrecordable_calls_are_refused(hip_available):
    pos, ctx = 64, 2048
    be = backend(1, ctx + 64, F16)
    L = N.lib()
    try:
        kb, vb = cache_rows(13, ctx)
        be.UploadKv(0, 0, ctx, kb, vb)
        q, k, v, qnw, knw = new_token(13, 0, "gamma")
        be.graph_begin()
        # host pointers synchronise: refused, and the recording is spoiled
        with pytest.raises(N.InvalidOperationError):
            be.DecodeAttention(0, pos, q[0], k[0], v[0], qnw, knw)
        assert L.hymt_sync(be.handle) == N.HYMT_E_STATE
        assert L.hymt_graph_begin(be.handle) == N.HYMT_E_STATE  # already open
        with pytest.raises(N.InvalidOperationError):
            be.graph_end()
        # a device-pointer call whose workspace would grow is refused too: a
        # 64-token prefill over 2048 cached positions splits its kv ranges
        # and needs the split workspace, which no call has allocated yet
        dq, dk, dv = dev_inputs(be, [q, k, v])
        dout = be.alloc(q.nbytes)
        qp, kp, vp = new_token(13, 1, None, seq=64)[:3]
        dqp, dkp, dvp = dev_inputs(be, [qp, kp, vp])
        doutp = be.alloc(qp.nbytes)
        be.decode_dev(0, pos, dq, dk, dv, None, None, dout)
        be.sync()
        be.graph_begin()
        with pytest.raises(N.InvalidOperationError) as e:
            be.prefill_dev(0, ctx, 64, dqp, dkp, dvp, F32, None, None, doutp)
        assert "workspace growth" in str(e.value)
        with pytest.raises(N.InvalidOperationError):
            be.graph_end()
        for p in (dqp, dkp, dvp, doutp):
            be.free(p)
        # an argument error records nothing and leaves the recording usable
        be.graph_begin()
        with pytest.raises(N.ArgumentError):
            be.decode_dev(7, pos, dq, dk, dv, None, None, dout)
        be.decode_dev(0, pos, dq, dk, dv, None, None, dout)
        g = be.graph_end()
        be.graph_launch(g)
        be.sync()
        be.graph_destroy(g)
        # misaligned device tensors are rejected before any work
        with pytest.raises(N.ArgumentError):
            be.decode_dev(0, pos, dq + 4, dk, dv, None, None, dout)
        for p in (dq, dk, dv, dout):
            be.free(p)
    finally:
        be.Dispose()


def test_recording_refused_after_buffer_growth(hip_available):
    """A recording replays the addresses of the context buffers it captured.
    Growing one of them afterwards (here the prefill split workspace, by an
    eager 64-token prefill over 2048 cached positions) makes
    hymt_graph_launch refuse the old recording instead of replaying accesses
    of freed memory; a new recording runs."""
    pos, ctx = 64, 2048
    be = backend(1, ctx + 64, F16)
    L = N.lib()
    try:
        kb, vb = cache_rows(14, ctx)
        be.UploadKv(0, 0, ctx, kb, vb)
        q, k, v, qnw, knw = new_token(14, 0, "gamma")
        dq, dk, dv = dev_inputs(be, [q, k, v])
        dout = be.alloc(q.nbytes)
        be.decode_dev(0, pos, dq, dk, dv, None, None, dout)
        be.sync()
        be.graph_begin()
        be.decode_dev(0, pos, dq, dk, dv, None, None, dout)
        g = be.graph_end()
        be.graph_launch(g)
        be.sync()
        ref = be.download(np.empty(HQ * D, np.float32), dout)
        qp, kp, vp = new_token(14, 1, None, seq=64)[:3]
        dqp, dkp, dvp = dev_inputs(be, [qp, kp, vp])
        doutp = be.alloc(qp.nbytes)
        be.prefill_dev(0, ctx, 64, dqp, dkp, dvp, F32, None, None, doutp)  # the workspace grows
        be.sync()
        for p in (dqp, dkp, dvp, doutp):
            be.free(p)
        assert L.hymt_graph_launch(be.handle, g) == N.HYMT_E_STATE
        assert b"record it again" in L.hymt_last_error()
        be.graph_destroy(g)
        be.decode_dev(0, pos, dq, dk, dv, None, None, dout)  # row pos rewritten as before
        be.graph_begin()
        be.decode_dev(0, pos, dq, dk, dv, None, None, dout)
        g = be.graph_end()
        be.upload(dout, np.zeros_like(q))
        be.graph_launch(g)
        be.sync()
        assert np.array_equal(be.download(np.empty(HQ * D, np.float32), dout), ref)
        be.graph_destroy(g)
        for p in (dq, dk, dv, dout):
            be.free(p)
    finally:
        be.Dispose()
