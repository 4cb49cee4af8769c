"""C ABI of libhymt_hip.so without a GPU: every declared symbol is exported,
argument and state errors come back as status codes, and the page table of a
host-only context (HYMT_DEVICE_NONE) follows the paged-KV rules."""
import ctypes
import os
import re

import numpy as np
import pytest

from hymt2sharp_amd import _native as N
from hymt2sharp_amd.backend import ArgumentError, InvalidOperationError, NotSupportedError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hymt_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(hymt_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 19
    lib = ctypes.CDLL(N.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding declares each of them
    assert set(names) - {"hymt_last_error"} <= set(N.SIGNATURES)


def test_abi_version():
    assert N.lib().hymt_abi_version() == 1


def host_ctx(max_tokens=1000, dtype=N.BF16):
    L = N.lib()
    h = ctypes.c_void_p()
    N.check(L.hymt_create(N.DEVICE_NONE, ctypes.byref(h)))
    N.check(L.hymt_set_attn_config(h, 16, 4, 128, 128, 10000.0, 1e-6))
    N.check(L.hymt_kv_create(h, 2, max_tokens, dtype))
    return L, h


def info(L, h):
    a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    N.check(L.hymt_kv_info(h, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
    return a.value, b.value, c.value


def page(L, h, b):
    p = ctypes.c_int()
    N.check(L.hymt_kv_page(h, b, ctypes.byref(p)))
    return p.value


def test_null_context_and_bad_arguments():
    L = N.lib()
    assert L.hymt_kv_set_len(None, 0) == N.HYMT_E_ARG
    assert b"null context" in L.hymt_last_error()
    assert L.hymt_destroy(None) == N.HYMT_OK
    assert L.hymt_create(0, None) == N.HYMT_E_ARG


def test_config_validation():
    L = N.lib()
    h = ctypes.c_void_p()
    N.check(L.hymt_create(N.DEVICE_NONE, ctypes.byref(h)))
    try:
        assert L.hymt_kv_create(h, 1, 64, N.BF16) == N.HYMT_E_STATE  # config first
        assert L.hymt_set_attn_config(h, 16, 5, 128, 128, 1e4, 1e-6) == N.HYMT_E_ARG
        assert L.hymt_set_attn_config(h, 16, 4, 64, 64, 1e4, 1e-6) == N.HYMT_E_UNSUPPORTED
        assert L.hymt_set_attn_config(h, 16, 16, 128, 128, 1e4, 1e-6) == N.HYMT_E_UNSUPPORTED
        assert L.hymt_set_attn_config(h, 16, 4, 128, 127, 1e4, 1e-6) == N.HYMT_E_ARG
        N.check(L.hymt_set_attn_config(h, 16, 4, 128, 128, 1e4, 1e-6))
        assert L.hymt_kv_create(h, 0, 64, N.BF16) == N.HYMT_E_ARG
        assert L.hymt_kv_create(h, 1, 64, 7) == N.HYMT_E_ARG
        N.check(L.hymt_kv_create(h, 1, 64, N.F16))
        assert L.hymt_kv_create(h, 1, 64, N.F16) == N.HYMT_E_STATE
        assert L.hymt_set_attn_config(h, 16, 4, 128, 128, 1e4, 1e-6) == N.HYMT_E_STATE
    finally:
        L.hymt_destroy(h)


def test_pages_round_up_and_map_on_write():
    L, h = host_ctx(1000)
    try:
        assert info(L, h) == (1024, 16, 0)
        N.check(L.hymt_kv_map(h, 0, 1))
        assert info(L, h)[2] == 1 and page(L, h, 0) == 0
        N.check(L.hymt_kv_map(h, 60, 10))  # crosses into block 1
        assert info(L, h)[2] == 2 and page(L, h, 1) == 1
        N.check(L.hymt_kv_map(h, 0, 128))  # already mapped: no change
        assert info(L, h)[2] == 2
        assert page(L, h, 2) == -1
    finally:
        L.hymt_destroy(h)


def test_capacity_errors():
    L, h = host_ctx(128)
    try:
        assert L.hymt_kv_map(h, 100, 29) == N.HYMT_E_CAPACITY
        assert b"capacity" in L.hymt_last_error()
        N.check(L.hymt_kv_map(h, 0, 128))
        q = np.zeros(2048, np.float32)
        k = np.zeros(512, np.float32)
        p = q.ctypes.data_as(ctypes.c_void_p)
        pk = k.ctypes.data_as(ctypes.c_void_p)
        assert L.hymt_attn_decode(h, 0, 128, p, pk, pk, None, None, p, 0) == N.HYMT_E_CAPACITY
        assert L.hymt_attn_prefill(h, 0, 100, 29, p, pk, pk, 0, None, None, p, 0) == N.HYMT_E_CAPACITY
    finally:
        L.hymt_destroy(h)


def test_set_len_recycles_pages():
    L, h = host_ctx(64 * 8)
    try:
        N.check(L.hymt_kv_map(h, 0, 64 * 5))
        assert [page(L, h, b) for b in range(6)] == [0, 1, 2, 3, 4, -1]
        N.check(L.hymt_kv_set_len(h, 130))  # keeps blocks 0..2
        assert [page(L, h, b) for b in range(5)] == [0, 1, 2, -1, -1]
        assert info(L, h)[2] == 3
        N.check(L.hymt_kv_map(h, 192, 128))  # blocks 3, 4 reuse freed pages
        assert sorted([page(L, h, 3), page(L, h, 4)]) == [3, 4]
        N.check(L.hymt_kv_map(h, 320, 64))  # block 5 takes a fresh page
        assert page(L, h, 5) == 5
        N.check(L.hymt_kv_set_len(h, 0))
        assert info(L, h)[2] == 0
        assert L.hymt_kv_set_len(h, -1) == N.HYMT_E_ARG
    finally:
        L.hymt_destroy(h)


def test_decode_requires_resident_prefix_and_device():
    L, h = host_ctx(256)
    try:
        q = np.zeros(2048, np.float32)
        k = np.zeros(512, np.float32)
        p = q.ctypes.data_as(ctypes.c_void_p)
        pk = k.ctypes.data_as(ctypes.c_void_p)
        # [0, 100) not written yet: KV gap (HunyuanDenseModel.cs:384-388)
        assert L.hymt_attn_decode(h, 0, 100, p, pk, pk, None, None, p, 0) == N.HYMT_E_STATE
        N.check(L.hymt_kv_map(h, 0, 100))
        assert L.hymt_attn_decode(h, 0, 100, p, pk, pk, None, None, p, 0) == N.HYMT_E_NO_DEVICE
        assert L.hymt_attn_decode(h, 2, 100, p, pk, pk, None, None, p, 0) == N.HYMT_E_ARG
        assert L.hymt_attn_decode(h, 0, 100, None, pk, pk, None, None, p, 0) == N.HYMT_E_ARG
        assert L.hymt_attn_prefill(h, 0, 0, 4, p, pk, pk, 5, None, None, p, 0) == N.HYMT_E_ARG
        assert L.hymt_sync(h) == N.HYMT_E_NO_DEVICE
    finally:
        L.hymt_destroy(h)


def test_graph_calls_need_a_device():
    L, h = host_ctx(64)
    try:
        g = ctypes.c_void_p()
        assert L.hymt_graph_begin(h) == N.HYMT_E_NO_DEVICE
        assert L.hymt_graph_end(h, ctypes.byref(g)) == N.HYMT_E_NO_DEVICE
        assert L.hymt_graph_launch(h, None) == N.HYMT_E_NO_DEVICE
        assert L.hymt_graph_begin(None) == N.HYMT_E_ARG
    finally:
        L.hymt_destroy(h)


def test_f32_cache_has_no_prefill():
    L, h = host_ctx(128, N.F32)
    try:
        q = np.zeros(2048, np.float32)
        p = q.ctypes.data_as(ctypes.c_void_p)
        assert L.hymt_attn_prefill(h, 0, 0, 1, p, p, p, 0, None, None, p, 0) == N.HYMT_E_UNSUPPORTED
    finally:
        L.hymt_destroy(h)


def test_status_maps_to_reference_exceptions():
    with pytest.raises(ArgumentError):
        N.check(N.HYMT_E_ARG)
    with pytest.raises(NotSupportedError):
        N.check(N.HYMT_E_CAPACITY)
    with pytest.raises(InvalidOperationError):
        N.check(N.HYMT_E_STATE)


def test_backend_factory_names(monkeypatch):
    from hymt2sharp_amd import create_backend
    assert create_backend("cpu") is None
    with pytest.raises(ArgumentError):
        create_backend("metal")
    monkeypatch.setenv("HYMT_BACKEND", "cpu")
    assert create_backend() is None


def test_misaligned_device_pointers_are_refused():
    """Device-pointer decode and prefill (packed and strided) refuse tensors
    that are not 16-byte aligned (the kernels load and store 16-byte vectors)
    before they look for a device, so the refusal shows on a host-only
    context; the pointers are never dereferenced."""
    L, h = host_ctx(256)
    try:
        ok, bad = 1 << 20, (1 << 20) + 8  # addresses only
        dev = N.FLAG_DEVICE_PTRS
        N.check(L.hymt_kv_map(h, 0, 64))
        # decode: every tensor argument, one at a time
        for i in range(6):
            args = [ok] * 6
            args[i] = bad
            q, k, v, qnw, knw, out = args
            assert L.hymt_attn_decode(h, 0, 10, q, k, v, qnw, knw, out, dev) == N.HYMT_E_ARG
            assert b"aligned" in L.hymt_last_error()
        assert L.hymt_attn_decode(h, 0, 10, ok, ok, ok, None, None, ok, dev) == N.HYMT_E_NO_DEVICE
        # packed prefill
        for i in range(6):
            args = [ok] * 6
            args[i] = bad
            q, k, v, qnw, knw, out = args
            assert L.hymt_attn_prefill(h, 0, 0, 16, q, k, v, N.BF16, qnw, knw, out, dev) == N.HYMT_E_ARG
            assert b"aligned" in L.hymt_last_error()
        assert L.hymt_attn_prefill(h, 0, 0, 16, ok, ok, ok, N.BF16, None, None, ok, dev) == N.HYMT_E_NO_DEVICE
        # strided prefill: base pointers checked, strides already multiples of 8
        ld = 3072
        for i in range(6):
            args = [ok] * 6
            args[i] = bad
            q, k, v, qnw, knw, out = args
            assert L.hymt_attn_prefill_ld(h, 0, 0, 16, q, ld, k, v, ld, N.BF16, qnw, knw, out, dev) == \
                N.HYMT_E_ARG
        assert L.hymt_attn_prefill_ld(h, 0, 0, 16, ok, ld, ok, ok, ld, N.BF16, None, None, ok, dev) == \
            N.HYMT_E_NO_DEVICE
        # host pointers are staged into aligned buffers: no refusal
        q = np.zeros(4096, np.float32)
        p = ctypes.c_void_p(q.ctypes.data + 4)
        assert L.hymt_attn_decode(h, 0, 10, p, p, p, None, None, p, 0) == N.HYMT_E_NO_DEVICE
    finally:
        L.hymt_destroy(h)


def test_model_prefill_refusals_without_device():
    """hymt_model_prefill needs a model; its argument checks come back as
    status codes."""
    L = N.lib()
    toks = np.zeros(4, np.int32)
    assert L.hymt_model_prefill(None, toks.ctypes.data_as(ctypes.c_void_p), 4, 0, None, 0) == N.HYMT_E_ARG
    L2, h = host_ctx(64)
    try:
        m = ctypes.c_void_p()
        # a model needs a device
        assert L2.hymt_model_create(h, 2, 2048, 6144, 512, 1e-5, ctypes.byref(m)) == N.HYMT_E_NO_DEVICE
    finally:
        L2.hymt_destroy(h)


def test_timing_readout_without_a_timer(monkeypatch):
    """hymt_timing_get / hymt_timing_reset: HYMT_E_STATE when the context does
    not time (a host-only context never does, whatever HYMT_HIP_TIMING says),
    HYMT_E_ARG for null arguments or a null context."""
    monkeypatch.setenv("HYMT_HIP_TIMING", "1")
    L, h = host_ctx(64)
    try:
        n, us = ctypes.c_long(), ctypes.c_double()
        assert L.hymt_timing_get(h, b"decode_attn", ctypes.byref(n), ctypes.byref(us)) == N.HYMT_E_STATE
        assert L.hymt_timing_reset(h) == N.HYMT_E_STATE
        assert L.hymt_timing_enable(h, 2) == N.HYMT_E_NO_DEVICE
        assert L.hymt_timing_get(h, None, ctypes.byref(n), ctypes.byref(us)) == N.HYMT_E_ARG
        assert L.hymt_timing_get(None, b"decode_attn", ctypes.byref(n), ctypes.byref(us)) == N.HYMT_E_ARG
    finally:
        L.hymt_destroy(h)
