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
    Weight.rows_dev          (Weight).RowInto           model.go:1034
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


_DTYPES = {"f32": ("float32",), "u8": ("uint8", "int8"), "u32": ("int32", "uint32"),
           "i32": ("int32",), "u16": ("int16", "uint16")}


def _dev(t, kind: str, numel: int, what: str):
    """Device pointer of tensor t after checking that it is a contiguous
    device tensor of the element kind with at least numel elements: a wrong
    tensor would otherwise become an out-of-bounds device access."""
    if not getattr(t, "is_cuda", False):
        raise ValueError(f"{what}: expected a device tensor")
    if str(t.dtype).replace("torch.", "") not in _DTYPES[kind]:
        raise ValueError(f"{what}: dtype {t.dtype}, expected {kind}")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{what}: {t.numel()} elements, need at least {numel}")
    return _dev_ptr(t)


def _host_f32(a, numel: int, what: str):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if a.size < numel:
        raise ValueError(f"{what}: {a.size} elements, need at least {numel}")
    return a


def _rows(t):
    return t.shape[0] if t.dim() == 2 else 1


def _stream(stream=None):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def available() -> bool:
    return bool(load().gllm_hip_available())


def stream_release(stream=None):
    """The caller will enqueue no more work on `stream` (default: torch's
    current stream): the calling thread's scratch for it is freed once it
    drains, except buffers a captured graph may still use."""
    call("gllm_hip_stream_release", _stream(stream))


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
        h = call_ptr("gllm_hip_weight_from_device", _dev(tensor, "u8", 0, "tensor"),
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
        x = _host_f32(x, self.cols, "matvec_into x")
        if out is None:
            out = np.empty(self.rows, np.float32)
        elif out.dtype != np.float32 or not out.flags.c_contiguous or out.size < self.rows:
            raise ValueError("matvec_into out: need a contiguous float32 array of rows elements")
        call("gllm_hip_matvec", self.handle, _np_ptr(x), _np_ptr(out))
        return out

    def matvec_batch(self, xs):
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        if xs.size % self.cols:
            raise ValueError("matvec_batch: xs is not a whole number of cols-wide rows")
        xs = xs.reshape(-1, self.cols)
        out = np.empty((xs.shape[0], self.rows), np.float32)
        call("gllm_hip_matvec_batch", self.handle, _np_ptr(xs), xs.shape[0], _np_ptr(out))
        return out

    def argmax_matvec(self, x, recent=None, penalty: float = 1.0) -> int:
        """Greedy token of W.x; with recent / penalty, after applyRepeatPenalty
        (sampling.go:136-153), as ArgmaxQ6KPenalized (internal/metal/
        metal_darwin.go:1175) takes them."""
        x = _host_f32(x, self.cols, "argmax_matvec x")
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
        p = _rows(xs)
        stride = out.shape[-1]
        if xs.shape[-1] != self.cols or stride < self.rows:
            raise ValueError(f"matvec_dev: xs (.., {xs.shape[-1]}) / out (.., {stride}) do not fit "
                             f"{self.rows}x{self.cols}")
        call("gllm_hip_matvec_dev", self.handle, _dev(xs, "f32", p * self.cols, "xs"), p,
             _dev(out, "f32", p * stride, "out"), stride, _stream(stream))
        return out

    def matvec_q8_dev(self, act, p, out, stream=None):
        """Row kernels only, against activations quantised by q8k_prepare_dev."""
        stride = out.shape[-1]
        if stride < self.rows:
            raise ValueError("matvec_q8_dev: out rows shorter than the weight's rows")
        call("gllm_hip_matvec_q8_dev", self.handle, _dev(act, "u8", act_bytes(self.cols, p), "act"),
             p, _dev(out, "f32", p * stride, "out"), stride, _stream(stream))
        return out

    def argmax_dev(self, x, token_out, stream=None, recent=None, penalty: float = 1.0):
        """recent: uint32/int32 device tensor of token ids, or None."""
        xp = _dev(x, "f32", self.cols, "x")
        tp = _dev(token_out, "u32", 1, "token_out")
        if recent is None and penalty == 1.0:
            call("gllm_hip_argmax_dev", self.handle, xp, tp, _stream(stream))
        else:
            n = 0 if recent is None else recent.numel()
            call("gllm_hip_argmax_penalized_dev", self.handle, xp,
                 _dev(recent, "u32", n, "recent") if n else None, n, float(penalty), tp,
                 _stream(stream))
        return token_out

    def lane_ints_dev(self, x, out, stream=None):
        call("gllm_hip_lane_ints_dev", self.handle, _dev(x, "f32", self.cols, "x"),
             _dev(out, "i32", self.rows * (self.cols // 256) * 8, "out"), _stream(stream))
        return out

    def rows_dev(self, ids, out, stream=None):
        """(Weight).RowInto (model.go:1034) for every id in the device
        tensor ids: out[i] = row ids[i] as f32 (ids must be < rows)."""
        n = ids.numel()
        call("gllm_hip_weight_rows_dev", self.handle, _dev(ids, "u32", n, "ids"), n,
             _dev(out, "f32", n * self.cols, "out"), _stream(stream))
        return out

    def download_dev(self, out, stream=None):
        call("gllm_hip_weight_download_dev", self.handle,
             _dev(out, "u8", self.rows * row_bytes(self.type, self.cols), "out"), _stream(stream))
        return out


def matvec_multi_dev(weights, xs, outs, stream=None):
    n = len(weights)
    p = _rows(xs)
    for w, o in zip(weights, outs):
        if xs.shape[-1] != w.cols or o.shape[-1] < w.rows:
            raise ValueError("matvec_multi_dev: xs / out shapes do not fit a weight")
    hs = (C.c_void_p * n)(*[w.handle for w in weights])
    ps = (C.c_void_p * n)(*[_dev(o, "f32", p * o.shape[-1], "out").value for o in outs])
    strides = (C.c_int * n)(*[o.shape[-1] for o in outs])
    call("gllm_hip_matvec_multi_dev", n, hs, _dev(xs, "f32", p * weights[0].cols, "xs"), p, ps,
         strides, _stream(stream))


def swiglu_down_dev(gate: Weight, up: Weight, down: Weight, x, out, stream=None):
    """down . siluMulF32(gate . x, up . x) for one token (ForwardBodyInto's
    FFN, model.go:2780-2800), gate/up routed as tryMatvec2Into routes them."""
    if gate.cols != up.cols or gate.rows != up.rows or down.cols != gate.rows:
        raise ValueError("swiglu_down_dev: gate / up / down shapes do not chain")
    call("gllm_hip_swiglu_down_dev", gate.handle, up.handle, down.handle,
         _dev(x, "f32", gate.cols, "x"), _dev(out, "f32", down.rows, "out"), _stream(stream))
    return out


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
    p = _rows(xs)
    cols = xs.shape[-1]
    call("gllm_hip_q8k_prepare_dev", _dev(xs, "f32", p * cols, "xs"), cols, p,
         _dev(act, "u8", act_bytes(cols, p), "act"), _stream(stream))
    return act


def q8k_quantize_dev(x, q8_out, scales_out, stream=None):
    p = _rows(x)
    cols = x.shape[-1]
    call("gllm_hip_q8k_quantize_dev", _dev(x, "f32", p * cols, "x"), cols, p,
         _dev(q8_out, "u8", p * cols, "q8_out"), _dev(scales_out, "f32", p * (cols // 256), "scales"),
         _stream(stream))


def quantize_rows_dev(qtype, src, dst, stream=None):
    rows, cols = src.shape
    call("gllm_hip_quantize_rows_dev", qtype, _dev(src, "f32", rows * cols, "src"), rows, cols,
         _dev(dst, "u8", rows * row_bytes(qtype, cols), "dst"), _stream(stream))
    return dst


def fill_normal_dev(out, seed: int, std: float, stream=None):
    call("gllm_hip_fill_normal_dev", _dev(out, "f32", 0, "out"), out.numel(), seed, std,
         _stream(stream))
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
        k = _host_f32(k, self.kv_dim_k, "store_kv k")
        v = _host_f32(v, self.kv_dim_v, "store_kv v")
        call("gllm_hip_kv_store", self.handle, layer, pos, _np_ptr(k), _np_ptr(v))

    def store_kv_dev(self, layer, pos, k, v, stream=None):
        call("gllm_hip_kv_store_dev", self.handle, layer, pos, _dev(k, "f32", self.kv_dim_k, "k"),
             _dev(v, "f32", self.kv_dim_v, "v"), _stream(stream))

    def attend_head_group(self, layer, kvh, queries, q_heads, hd, vd, start, end, scale,
                          softcap=0.0):
        queries = _host_f32(queries, q_heads * hd, "attend_head_group queries")
        out = np.empty(q_heads * vd, np.float32)
        call("gllm_hip_attend_group", self.handle, layer, kvh, _np_ptr(queries), q_heads, hd, vd,
             start, end, scale, softcap, _np_ptr(out))
        return out

    def attend_dev(self, layer, q, n_heads, n_kv_heads, hd, start, end, scale, out,
                   mode=ATTN_EXACT, stream=None):
        call("gllm_hip_attend_dev", self.handle, layer, _dev(q, "f32", n_heads * hd, "q"), n_heads,
             n_kv_heads, hd, start, end, scale, mode, _dev(out, "f32", n_heads * hd, "out"),
             _stream(stream))
        return out
