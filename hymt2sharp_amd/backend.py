"""Python mirror of the reference's backend plugin surface for the attention
path, over the C ABI of libhymt_hip.so.

HipBackend follows IComputeBackend (Backends/IComputeBackend.cs:14-88) for
the members this path owns -- Name, SupportsPrefill, UploadKv, SetCacheLen,
the device block store (SupportsBlockStore, DeviceBlockTokens, HarvestPrefix,
RestorePrefix), Dispose -- and adds the per-layer attention unit the reference runs inside
ForwardStep (DecodeAttention / PrefillAttention, HunyuanDenseModel.Decode.cs:64-101,
HunyuanDenseModel.Prefill.cs:38-89).  create_backend mirrors
BackendFactory.Create (Backends/BackendFactory.cs:15-44) with the "hip" name
added.  Errors raise the Python counterparts of the reference's exceptions.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _native as N
from ._native import (ArgumentError, InvalidOperationError, NotSupportedError,  # noqa: F401
                      PlatformNotSupportedError)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


class HipBackend:
    """`HipBackend : IComputeBackend` for the attention path on one MI355X."""

    Name = "hip"
    SupportsPrefill = True
    SupportsBlockStore = True
    DeviceBlockTokens = N.PAGE_TOKENS

    def __init__(self, device: int = 0):
        self._lib = N.lib()
        h = ctypes.c_void_p()
        N.check(self._lib.hymt_create(device, ctypes.byref(h)))
        self._h = h
        self.device = device
        self.heads = self.kv_heads = self.head_dim = 0

    # -- configuration (ModelConfig, ModelConfig.cs:21-51) --------------------
    def configure(self, heads=16, kv_heads=4, head_dim=128, rope_dim=None, rope_base=10000.0,
                  eps=1e-6):
        rope_dim = head_dim if rope_dim is None else rope_dim
        N.check(self._lib.hymt_set_attn_config(self._h, heads, kv_heads, head_dim, rope_dim,
                                               rope_base, eps))
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.rope_dim, self.rope_base, self.eps = rope_dim, rope_base, eps
        return self

    def create_cache(self, layers: int, max_tokens: int, kv_dtype: int = N.BF16):
        """KV part of LoadModel (MetalBackend.cs:164-181)."""
        N.check(self._lib.hymt_kv_create(self._h, layers, max_tokens, kv_dtype))
        self.layers, self.kv_dtype = layers, kv_dtype
        return self

    @property
    def handle(self):
        return self._h

    def cache_info(self):
        a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        N.check(self._lib.hymt_kv_info(self._h, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
        return {"max_tokens": a.value, "pages_total": b.value, "pages_mapped": c.value}

    def page_of(self, block: int) -> int:
        p = ctypes.c_int()
        N.check(self._lib.hymt_kv_page(self._h, block, ctypes.byref(p)))
        return p.value

    # -- IComputeBackend members ------------------------------------------
    def UploadKv(self, layer: int, pos: int, length: int, k_bf16: np.ndarray, v_bf16: np.ndarray):
        """IComputeBackend.UploadKv (IComputeBackend.cs:31-38): rows [pos, pos+len)
        of the model's flat bf16 caches (row j at j*kv_stride)."""
        k = np.ascontiguousarray(k_bf16, dtype=np.uint16)
        v = np.ascontiguousarray(v_bf16, dtype=np.uint16)
        stride = self.kv_heads * self.head_dim
        if k.size < (pos + length) * stride or v.size < (pos + length) * stride:
            raise ArgumentError(N.HYMT_E_ARG, "cache arrays shorter than pos+len rows")
        N.check(self._lib.hymt_kv_upload(self._h, layer, pos, length, _ptr(k), _ptr(v)))

    def SetCacheLen(self, length: int):
        """IComputeBackend.SetCacheLen (IComputeBackend.cs:82-87)."""
        N.check(self._lib.hymt_kv_set_len(self._h, length))

    def HarvestPrefix(self, tokens, block_tokens: int):
        """IComputeBackend.HarvestPrefix (IComputeBackend.cs:49-87; Metal's,
        MetalBackend.cs:330-356): pin every full mapped block of `tokens`."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        N.check(self._lib.hymt_kv_harvest(self._h, _ptr(t), t.size, block_tokens))

    def RestorePrefix(self, tokens, block_tokens: int) -> int:
        """IComputeBackend.RestorePrefix (MetalBackend.cs:358-382): map the
        longest stored run of full blocks of `tokens`; tokens restored."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        n = ctypes.c_int()
        N.check(self._lib.hymt_kv_restore(self._h, _ptr(t), t.size, block_tokens, ctypes.byref(n)))
        return n.value

    def store_info(self):
        e, f = ctypes.c_int(), ctypes.c_int()
        N.check(self._lib.hymt_kv_store_info(self._h, ctypes.byref(e), ctypes.byref(f)))
        return {"entries": e.value, "pages_free": f.value}

    def MapRange(self, pos: int, length: int):
        N.check(self._lib.hymt_kv_map(self._h, pos, length))

    def ReadKv(self, layer: int, pos: int, length: int):
        """Rows [pos, pos+len) of one layer as fp32 [len][kv_heads*head_dim]."""
        stride = self.kv_heads * self.head_dim
        k = np.empty((length, stride), dtype=np.float32)
        v = np.empty((length, stride), dtype=np.float32)
        N.check(self._lib.hymt_kv_read(self._h, layer, pos, length, _ptr(k), _ptr(v)))
        return k, v

    # -- attention unit ---------------------------------------------------
    def DecodeAttention(self, layer: int, pos: int, q, k, v, qnw=None, knw=None) -> np.ndarray:
        """Attention of DecodeAttention (Decode.cs:79-95): RoPE, QK norm, append,
        softmax(qK^T/sqrt(D))V over [0, pos].  Host arrays in, out[heads*head_dim]."""
        q, k, v, qnw, knw = map(_f32, (q, k, v, qnw, knw))
        out = np.empty(self.heads * self.head_dim, dtype=np.float32)
        N.check(self._lib.hymt_attn_decode(self._h, layer, pos, _ptr(q), _ptr(k), _ptr(v),
                                           _ptr(qnw), _ptr(knw), _ptr(out), 0))
        return out

    def PrefillAttention(self, layer: int, pos: int, q, k, v, qnw=None, knw=None,
                         io_dtype: int = N.F32) -> np.ndarray:
        """Attention of PrefillAttention (Prefill.cs:53-83) for one chunk.
        q [seq][heads*D], k/v [seq][kv_heads*D] as fp32 (or bf16 bit patterns
        when io_dtype is BF16).  Returns out[seq][heads*D] fp32."""
        if io_dtype == N.BF16:
            q, k, v = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v))
        else:
            q, k, v = map(_f32, (q, k, v))
        qnw, knw = _f32(qnw), _f32(knw)
        seq = q.size // (self.heads * self.head_dim)
        out = np.empty((seq, self.heads * self.head_dim), dtype=np.float32)
        N.check(self._lib.hymt_attn_prefill(self._h, layer, pos, seq, _ptr(q), _ptr(k), _ptr(v),
                                            io_dtype, _ptr(qnw), _ptr(knw), _ptr(out), 0))
        return out

    # -- device-pointer variants (activations resident in HBM) -------------
    def decode_dev(self, layer, pos, q, k, v, qnw, knw, out):
        N.check(self._lib.hymt_attn_decode(self._h, layer, pos, q, k, v, qnw, knw, out,
                                           N.FLAG_DEVICE_PTRS))

    def prefill_dev(self, layer, pos, seq, q, k, v, io_dtype, qnw, knw, out):
        N.check(self._lib.hymt_attn_prefill(self._h, layer, pos, seq, q, k, v, io_dtype, qnw, knw,
                                            out, N.FLAG_DEVICE_PTRS))

    def prefill_dev_ld(self, layer, pos, seq, q, q_ld, k, v, kv_ld, io_dtype, qnw, knw, out):
        """prefill_dev over rows q_ld (k, v: kv_ld) elements apart."""
        N.check(self._lib.hymt_attn_prefill_ld(self._h, layer, pos, seq, q, q_ld, k, v, kv_ld, io_dtype,
                                               qnw, knw, out, N.FLAG_DEVICE_PTRS))

    def alloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        N.check(self._lib.hymt_dev_alloc(self._h, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, p):
        N.check(self._lib.hymt_dev_free(self._h, p))

    def upload(self, dptr, arr: np.ndarray):
        a = np.ascontiguousarray(arr)
        N.check(self._lib.hymt_memcpy(self._h, dptr, _ptr(a), a.nbytes, 0))

    def download(self, arr: np.ndarray, dptr):
        N.check(self._lib.hymt_memcpy(self._h, _ptr(arr), dptr, arr.nbytes, 1))
        return arr

    def sync(self):
        N.check(self._lib.hymt_sync(self._h))

    # -- per-kernel timing (HYMT_HIP_TIMING=1 or quiet at creation) -------
    def timing(self, kernel: str):
        """(count, summed microseconds) of `kernel` over the timed calls."""
        n, us = ctypes.c_long(), ctypes.c_double()
        N.check(self._lib.hymt_timing_get(self._h, kernel.encode(), ctypes.byref(n), ctypes.byref(us)))
        return n.value, us.value

    def timing_enable(self, mode: int):
        """0 off (totals kept), 1 time and print per call, 2 time quietly."""
        N.check(self._lib.hymt_timing_enable(self._h, mode))

    def timing_reset(self):
        N.check(self._lib.hymt_timing_reset(self._h))

    # ---- quantized weights (the weight half of LoadModel, IComputeBackend.cs:25-29)
    def weight_upload(self, wtype: int, rows: int, cols: int, data) -> int:
        """Upload a rows x cols matrix given as rows of GGUF blocks; returns a
        handle for gemv / weight_free."""
        raw = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
        h = ctypes.c_void_p()
        N.check(self._lib.hymt_weight_upload(self._h, wtype, rows, cols, _ptr(raw), raw.nbytes,
                                             ctypes.byref(h)))
        return h.value

    def weight_free(self, w):
        N.check(self._lib.hymt_weight_free(self._h, w))

    def weight_info(self, w) -> dict:
        t, r, c, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
        N.check(self._lib.hymt_weight_info(w, ctypes.byref(t), ctypes.byref(r), ctypes.byref(c),
                                           ctypes.byref(b)))
        return {"type": t.value, "rows": r.value, "cols": c.value, "device_bytes": b.value}

    def gemv(self, w, x_dev, y_dev, accumulate: bool = False, rmsnorm=None, eps: float = 1e-6,
             swiglu: bool = False, swiglu_out: bool = False):
        """y (+)= W x' on device vectors (enqueued on the context's stream);
        x' = RMSNorm(x) * rmsnorm (a device pointer) or silu(gate) * up.
        swiglu_out: W is [gate; up] and y = silu(gate rows . x') * (up rows . x')."""
        flags = (N.GEMV_ACCUMULATE if accumulate else 0) | (N.GEMV_IN_RMSNORM if rmsnorm else 0) | \
                (N.GEMV_IN_SWIGLU if swiglu else 0) | (N.GEMV_OUT_SWIGLU if swiglu_out else 0)
        N.check(self._lib.hymt_gemv(self._h, w, x_dev, y_dev, flags, rmsnorm, eps))

    # ---- the model: IComputeBackend.LoadModel / ForwardStep (IComputeBackend.cs:25-47)
    def LoadModel(self, tensors: dict, config, max_tokens: int = 4096, kv_dtype: int = N.BF16,
                  prefill: bool = True):
        """tensors: GGUF name -> model.Tensor; config: model.ModelConfig.
        Uploads every weight, creates the KV cache, keeps activations on the
        device (hymt2sharp_amd/model.py).  prefill: also keep bf16 dense
        copies of the layer weights so that multi-token calls run as GEMMs."""
        from .model import DeviceModel
        if getattr(self, "_model", None) is not None:
            self._model.free()
            self._model = None
        self._model = DeviceModel(self, config, tensors, max_tokens, kv_dtype, prefill=prefill)
        return self

    def ForwardStep(self, tokens, pos: int) -> np.ndarray:
        """Logits of the last token after running `tokens` at positions pos..;
        the device KV holds [0, pos) before and [0, pos + len) after."""
        if getattr(self, "_model", None) is None:
            raise N.InvalidOperationError(N.HYMT_E_STATE, "LoadModel first")
        return self._model.forward(tokens, pos)

    def embed(self, w, row: int, out_dev):
        """out = row `row` of W, dequantized (device pointer)."""
        N.check(self._lib.hymt_embed(self._h, w, row, out_dev))

    # ---- prefill: dense weights, GEMMs and row kernels (device pointers)
    def weight_dense(self, w):
        """Give W a bf16 dense copy for gemm (synchronous)."""
        N.check(self._lib.hymt_weight_dense(self._h, w))

    def gemm(self, w, x_dev, m: int, y_dev, row0: int = 0, nrows: int | None = None,
             accumulate: bool = False, out_bf16: bool = False):
        """y[m][nrows] (+)= x[m][cols] . W[row0:row0+nrows]^T (x bf16; y fp32 or bf16)."""
        if nrows is None:
            nrows = self.weight_info(w)["rows"] - row0
        flags = (N.GEMM_ACCUMULATE if accumulate else 0) | (N.GEMM_OUT_BF16 if out_bf16 else 0)
        N.check(self._lib.hymt_gemm(self._h, w, row0, nrows, x_dev, m, y_dev, flags))

    def gemm_swiglu(self, gate, x_dev, m: int, act_dev, up=None):
        """act[m][f] = bf16(silu(g) u) with g, u the bf16 products of x over the
        gate and up rows (gate = one [gate; up] weight with up None, or the gate
        rows with up the up rows), fused; NotSupportedError where the fused
        launch would not give the bits of gemm(out_bf16) + rows_swiglu_bf16."""
        N.check(self._lib.hymt_gemm_swiglu(self._h, gate, up, x_dev, m, act_dev))

    def embed_rows(self, w, rows, out_dev):
        r = np.ascontiguousarray(rows, dtype=np.int32)
        N.check(self._lib.hymt_embed_rows(self._h, w, _ptr(r), r.size, out_dev))

    def rows_rmsnorm(self, x_dev, m: int, n: int, norm_w_dev, eps: float, out_dev):
        N.check(self._lib.hymt_rows_rmsnorm(self._h, x_dev, m, n, norm_w_dev, eps, out_dev))

    def rows_swiglu(self, gu_dev, m: int, n: int, out_dev):
        N.check(self._lib.hymt_rows_swiglu(self._h, gu_dev, m, n, out_dev))

    def rows_swiglu_bf16(self, gu_dev, m: int, n: int, out_dev):
        N.check(self._lib.hymt_rows_swiglu_bf16(self._h, gu_dev, m, n, out_dev))

    def to_bf16(self, x_dev, count: int, out_dev):
        N.check(self._lib.hymt_to_bf16(self._h, x_dev, count, out_dev))

    def stream(self) -> int:
        s = ctypes.c_void_p()
        N.check(self._lib.hymt_get_stream(self._h, ctypes.byref(s)))
        return s.value

    # -- recorded call sequences (HIP graphs) ----------------------------
    def graph_begin(self):
        """Start recording device-pointer calls on the context's stream
        (the recorded decode command buffer of VulkanBackend.cs:400-568)."""
        N.check(self._lib.hymt_graph_begin(self._h))

    def graph_end(self) -> int:
        g = ctypes.c_void_p()
        N.check(self._lib.hymt_graph_end(self._h, ctypes.byref(g)))
        return g.value

    def graph_launch(self, g: int):
        N.check(self._lib.hymt_graph_launch(self._h, g))

    def graph_destroy(self, g: int):
        N.check(self._lib.hymt_graph_destroy(self._h, g))

    # -- IDisposable ------------------------------------------------------
    def Dispose(self):
        if getattr(self, "_model", None) is not None and getattr(self, "_h", None):
            self._model.free()
            self._model = None
        if self._h:
            N.check(self._lib.hymt_destroy(self._h))
            self._h = None

    close = Dispose

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.Dispose()

    def __del__(self):
        try:
            self.Dispose()
        except Exception:
            pass


def device_count() -> int:
    n = ctypes.c_int()
    N.check(N.lib().hymt_device_count(ctypes.byref(n)))
    return n.value


def create_backend(preference: str | None = None):
    """BackendFactory.Create (BackendFactory.cs:15-44) with "hip" added.

    An explicit "hip" constructs the backend and raises if it cannot run;
    "auto" returns a HipBackend when a device works and None (the CPU engine)
    otherwise; "cpu" returns None.
    """
    p = (preference if preference is not None else os.environ.get("HYMT_BACKEND", "auto"))
    p = p.strip().lower()
    if p in ("", "auto"):
        try:
            if device_count() > 0:
                return HipBackend(int(os.environ.get("HYMT_HIP_DEVICE", "0")))
        except Exception:
            pass
        return None
    if p == "cpu":
        return None
    if p == "hip":
        return HipBackend(int(os.environ.get("HYMT_HIP_DEVICE", "0")))
    raise ArgumentError(N.HYMT_E_ARG, f"unknown backend '{p}' (expected auto|cpu|hip)")
