"""Python mirror of the reference's matvec / attention call surface over the
C ABI (include/gllm_hip.h).  Names follow the Go API they stand in for:

    Weight.matvec_into       (Weight).MatvecInto        model.go:670
    Weight.argmax_matvec     (Weight).ArgmaxMatvec      model.go:754
    matvec_q4k_into          MatvecQ4KInto              simd.go:261
    matvec_q6k_into          MatvecQ6KInto              simd.go:413
    matvec_q8_0_into         MatvecQ8_0Into             simd.go:204
    matvec2_into / matvec3_into   MatvecQ4K2IntoWithXSums simd.go:295,
                             Q4KMatvec3IntoWithXSums    metal.go:14
    matvec_batch             matvecBatchQ8              kernels_amd64.go:470
    KVCacheF16.store_kv      (*KVCache).storeKV         model.go:1466
    KVCacheF16.attend_head_group (*KVCache).attendHeadGroup model.go:1516

Host arrays are numpy; device arrays are torch tensors on a ROCm device (torch
supplies device memory and streams only -- every computation is a HIP kernel
of libgllm_hip).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import (TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, ATTN_EXACT, ATTN_SPLITK, call, call_ptr,
                   load)



def row_bytes(qtype: int, cols: int) -> int:
    """GGMLType.DataSize for one row (gguf.go:241-297)."""
    return int(load().gllm_hip_ggml_data_size(int(qtype), int(cols)))


def _np_ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _dev_ptr(t):
    return C.c_void_p(t.data_ptr())


def _stream(stream=None):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def available() -> bool:
    return bool(load().gllm_hip_available())


class Weight:
    """A quantized GGUF tensor resident in HBM (prepareMetalWeight, model.go:2454)."""

    def __init__(self, handle, qtype, rows, cols):
        self.handle = handle
        self.type, self.rows, self.cols = qtype, rows, cols

    @classmethod
    def from_host(cls, raw, qtype: int, rows: int, cols: int) -> "Weight":
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        h = call_ptr("gllm_hip_weight_new", _np_ptr(raw), raw.nbytes, qtype, rows, cols)
        return cls(h, qtype, rows, cols)

    @classmethod
    def from_device(cls, tensor, qtype: int, rows: int, cols: int, stream=None) -> "Weight":
        h = call_ptr("gllm_hip_weight_from_device", _dev_ptr(tensor),
                     tensor.numel() * tensor.element_size(), qtype, rows, cols, _stream(stream))
        return cls(h, qtype, rows, cols)

    def release(self):
        if self.handle:
            load().gllm_hip_weight_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    # host-pointer forms ----------------------------------------------------
    def matvec_into(self, x, out=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.size < self.cols:
            raise ValueError("x shorter than cols")
        if out is None:
            out = np.empty(self.rows, np.float32)
        call("gllm_hip_matvec", self.handle, _np_ptr(x), _np_ptr(out))
        return out

    def matvec_batch(self, xs):
        xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1, self.cols)
        out = np.empty((xs.shape[0], self.rows), np.float32)
        call("gllm_hip_matvec_batch", self.handle, _np_ptr(xs), xs.shape[0], _np_ptr(out))
        return out

    def argmax_matvec(self, x, recent=None, penalty: float = 1.0) -> int:
        """Greedy token of W.x; with recent / penalty, after applyRepeatPenalty
        (sampling.go:136-153), as ArgmaxQ6KPenalized (internal/metal/
        metal_darwin.go:1175) takes them."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        tok = C.c_uint32(0)
        if recent is None and penalty == 1.0:
            call("gllm_hip_argmax", self.handle, _np_ptr(x), C.byref(tok))
        else:
            rec = np.ascontiguousarray(recent if recent is not None else [], dtype=np.uint32)
            call("gllm_hip_argmax_penalized", self.handle, _np_ptr(x),
                 _np_ptr(rec) if rec.size else None, rec.size, float(penalty), C.byref(tok))
        return int(tok.value)

    # device forms ------------------------------------------------------------
    def matvec_dev(self, xs, out, stream=None):
        """xs: (p, cols) float32 device tensor; out: (p, >= rows) float32."""
        p = xs.shape[0] if xs.dim() == 2 else 1
        stride = out.shape[-1]
        call("gllm_hip_matvec_dev", self.handle, _dev_ptr(xs), p, _dev_ptr(out), stride,
             _stream(stream))
        return out

    def matvec_q8_dev(self, act, p, out, stream=None):
        """Row kernels only, against activations quantised by q8k_prepare_dev."""
        call("gllm_hip_matvec_q8_dev", self.handle, _dev_ptr(act), p, _dev_ptr(out),
             out.shape[-1], _stream(stream))
        return out

    def argmax_dev(self, x, token_out, stream=None, recent=None, penalty: float = 1.0):
        """recent: uint32/int32 device tensor of token ids, or None."""
        if recent is None and penalty == 1.0:
            call("gllm_hip_argmax_dev", self.handle, _dev_ptr(x), _dev_ptr(token_out),
                 _stream(stream))
        else:
            n = 0 if recent is None else recent.numel()
            call("gllm_hip_argmax_penalized_dev", self.handle, _dev_ptr(x),
                 _dev_ptr(recent) if n else None, n, float(penalty), _dev_ptr(token_out),
                 _stream(stream))
        return token_out

    def lane_ints_dev(self, x, out, stream=None):
        call("gllm_hip_lane_ints_dev", self.handle, _dev_ptr(x), _dev_ptr(out), _stream(stream))
        return out

    def download_dev(self, out, stream=None):
        call("gllm_hip_weight_download_dev", self.handle, _dev_ptr(out), _stream(stream))
        return out


def matvec_multi_dev(weights, xs, outs, stream=None):
    n = len(weights)
    hs = (C.c_void_p * n)(*[w.handle for w in weights])
    ps = (C.c_void_p * n)(*[o.data_ptr() for o in outs])
    strides = (C.c_int * n)(*[o.shape[-1] for o in outs])
    p = xs.shape[0] if xs.dim() == 2 else 1
    call("gllm_hip_matvec_multi_dev", n, hs, _dev_ptr(xs), p, ps, strides, _stream(stream))


def _matvec_into(qtype, data, x, rows, cols, out):
    w = Weight.from_host(data, qtype, rows, cols)
    try:
        return w.matvec_into(x, out)
    finally:
        w.release()


def matvec_q4k_into(data, x, rows, cols, out=None):
    return _matvec_into(TYPE_Q4_K, data, x, rows, cols, out)


def matvec_q6k_into(data, x, rows, cols, out=None):
    return _matvec_into(TYPE_Q6_K, data, x, rows, cols, out)


def matvec_q8_0_into(data, x, rows, cols, out=None):
    return _matvec_into(TYPE_Q8_0, data, x, rows, cols, out)


def matvec2_into(a: Weight, b: Weight, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    oa, ob = np.empty(a.rows, np.float32), np.empty(b.rows, np.float32)
    call("gllm_hip_matvec2", a.handle, b.handle, _np_ptr(x), _np_ptr(oa), _np_ptr(ob))
    return oa, ob


def matvec3_into(a: Weight, b: Weight, c: Weight, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    oa, ob, oc = (np.empty(w.rows, np.float32) for w in (a, b, c))
    call("gllm_hip_matvec3", a.handle, b.handle, c.handle, _np_ptr(x), _np_ptr(oa),
         _np_ptr(ob), _np_ptr(oc))
    return oa, ob, oc


def act_bytes(cols: int, p: int = 1) -> int:
    """Bytes of the quantised-activation buffer for p rows of cols."""
    return int(load().gllm_hip_act_bytes(cols, p))


def q8k_prepare_dev(xs, act, stream=None):
    """acquireQ8 + xsums for p rows of xs into the device buffer `act`."""
    p = xs.shape[0] if xs.dim() == 2 else 1
    call("gllm_hip_q8k_prepare_dev", _dev_ptr(xs), xs.shape[-1], p, _dev_ptr(act), _stream(stream))
    return act


def q8k_quantize_dev(x, q8_out, scales_out, stream=None):
    p = x.shape[0] if x.dim() == 2 else 1
    cols = x.shape[-1]
    call("gllm_hip_q8k_quantize_dev", _dev_ptr(x), cols, p, _dev_ptr(q8_out),
         _dev_ptr(scales_out), _stream(stream))


def quantize_rows_dev(qtype, src, dst, stream=None):
    rows, cols = src.shape
    call("gllm_hip_quantize_rows_dev", qtype, _dev_ptr(src), rows, cols, _dev_ptr(dst),
         _stream(stream))
    return dst


def fill_normal_dev(out, seed: int, std: float, stream=None):
    call("gllm_hip_fill_normal_dev", _dev_ptr(out), out.numel(), seed, std, _stream(stream))
    return out


class KVCacheF16:
    """HBM-resident F16 KV cache (NewKVCacheF16, model.go:1396)."""

    def __init__(self, layers, kv_dim_k, kv_dim_v, max_len, handle=None, owned=True):
        self.layers, self.kv_dim_k, self.kv_dim_v, self.max_len = layers, kv_dim_k, kv_dim_v, max_len
        self.handle = handle or call_ptr("gllm_hip_kv_new", layers, kv_dim_k, kv_dim_v, max_len)
        self.owned = owned

    def release(self):
        if self.handle and self.owned:
            load().gllm_hip_kv_release(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def k_ptr(self, layer):
        return load().gllm_hip_kv_k_dev(self.handle, layer)

    def v_ptr(self, layer):
        return load().gllm_hip_kv_v_dev(self.handle, layer)

    def read(self, layer, pos0, n):
        """(K rows, V rows) of positions pos0..pos0+n-1 as f16 bit arrays."""
        k = np.empty((n, self.kv_dim_k), np.uint16)
        v = np.empty((n, self.kv_dim_v), np.uint16)
        call("gllm_hip_kv_read", self.handle, layer, pos0, n, _np_ptr(k), _np_ptr(v))
        return k, v

    def store_kv(self, layer, pos, k, v):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        call("gllm_hip_kv_store", self.handle, layer, pos, _np_ptr(k), _np_ptr(v))

    def store_kv_dev(self, layer, pos, k, v, stream=None):
        call("gllm_hip_kv_store_dev", self.handle, layer, pos, _dev_ptr(k), _dev_ptr(v),
             _stream(stream))

    def attend_head_group(self, layer, kvh, queries, q_heads, hd, vd, start, end, scale,
                          softcap=0.0):
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        out = np.empty(q_heads * vd, np.float32)
        call("gllm_hip_attend_group", self.handle, layer, kvh, _np_ptr(queries), q_heads, hd, vd,
             start, end, scale, softcap, _np_ptr(out))
        return out

    def attend_dev(self, layer, q, n_heads, n_kv_heads, hd, start, end, scale, out,
                   mode=ATTN_EXACT, stream=None):
        call("gllm_hip_attend_dev", self.handle, layer, _dev_ptr(q), n_heads, n_kv_heads, hd,
             start, end, scale, mode, _dev_ptr(out), _stream(stream))
        return out
