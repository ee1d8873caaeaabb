"""ctypes front end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke`` and
the ``cpu_baseline`` leg of ``bench.py`` -- never by the product package.
Each wrapper names the C routine it calls; the C file cites the reference
lines it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
Q4_0, Q4_1, Q2_K, Q3_K, Q5_K, MXFP4 = 2, 3, 10, 11, 13, 39
BF16 = 30
EXTRA_TYPES = (Q5_K, Q4_0, Q4_1, MXFP4, Q2_K, Q3_K)
GENERIC, AMD64 = 0, 1

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i, l, f = C.c_void_p, C.c_int, C.c_long, C.c_float
        sig = {
            "ref_f16_to_f32": (f, [C.c_uint16]),
            "ref_f32_to_f16": (C.c_uint16, [f]),
            "ref_f32_to_f16_row": (None, [vp, vp, l]),
            "ref_f16_to_f32_row": (None, [vp, vp, l]),
            "ref_round_to_even_f32": (f, [f]),
            "ref_q8k_quantize": (None, [vp, vp, vp, i]),
            "ref_xsums32": (None, [vp, vp, i, i]),
            "ref_xsums16": (None, [vp, vp, i, i, i]),
            "ref_q4k_dot": (f, [vp, vp, vp, vp, i, i]),
            "ref_q6k_dot": (f, [vp, vp, vp, vp, i, i]),
            "ref_q8_0_dot": (f, [vp, vp, vp, i, i]),
            "ref_q4k_dot_avx2": (f, [vp, vp, vp, vp, i]),
            "ref_q6k_dot_avx2": (f, [vp, vp, vp, vp, i]),
            "ref_q8_0_dot_avx2": (f, [vp, vp, vp, i]),
            "ref_lane_ints": (None, [i, vp, vp, i, vp]),
            "ref_row_dot_any": (f, [i, vp, vp, vp, vp, i, i]),
            "ref_type_supported": (i, [i]),
            "ref_row_bytes": (l, [i, i]),
            "ref_matvec": (i, [i, vp, vp, i, i, vp, i, i]),
            "ref_matvec_batch": (i, [i, vp, vp, i, i, i, vp, i, i]),
            "ref_float_dot_supported": (i, [i]),
            "ref_float_dot": (f, [i, vp, vp, i]),
            "ref_matvec_float": (i, [i, vp, vp, i, i, vp, i]),
            "ref_matvec_batch_fast": (i, [i, vp, vp, i, i, i, vp, i]),
            "ref_argmax_matvec": (C.c_uint32, [i, vp, vp, i, i, i, i]),
            "ref_argmax_finite": (C.c_uint32, [vp, l]),
            "ref_apply_repeat_penalty": (None, [vp, l, vp, i, f]),
            "ref_quantize_rows": (None, [i, vp, l, i, vp, i]),
            "ref_dequant_row": (None, [i, vp, i, vp]),
            "ref_dot_f32": (f, [vp, vp, l]),
            "ref_dot_f32_f16": (f, [vp, vp, l]),
            "ref_fast_exp": (f, [f]),
            "ref_silu_mul": (None, [vp, vp, vp, l]),
            "ref_rmsnorm": (None, [vp, vp, f, l, vp]),
            "ref_rope_inv_freq": (None, [f, i, vp]),
            "ref_rope_sincos": (None, [i, vp, i, vp, vp]),
            "ref_rope_apply": (None, [vp, i, i, i, vp, vp]),
            "ref_attend_group_f16": (None, [vp, vp, vp, i, l, l, i, i, i, i, f, vp]),
            "ref_llama_state_new": (vp, [vp, i]),
            "ref_llama_state_free": (None, [vp]),
            "ref_llama_set_fast": (None, [vp, i]),
            "ref_llama_set_repeat_penalty": (None, [vp, f, i]),
            "ref_llama_decode": (C.c_uint32, [vp, C.c_uint32, i, vp]),
            "ref_llama_prefill": (C.c_uint32, [vp, vp, i, i, i, vp]),
            "ref_llama_generate": (None, [vp, vp, i, i, i, vp]),
            "ref_llama_kcache": (vp, [vp, i]),
            "ref_llama_vcache": (vp, [vp, i]),
            "ref_num_threads": (i, []),
            "ref_has_avx2": (i, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


# ---- f16 -------------------------------------------------------------------
def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ref_f16_to_f32_row(_p(h), _p(out), h.size)
    return out


def f32_to_f16(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().ref_f32_to_f16_row(_p(x), _p(out), x.size)
    return out


# ---- activation quantisation ----------------------------------------------
def q8k_quantize(x):
    x = _f32(x)
    blocks = x.size // 256
    q8 = np.empty(blocks * 256, np.int8)
    sc = np.empty(blocks, np.float32)
    lib().ref_q8k_quantize(_p(x), _p(q8), _p(sc), blocks)
    return q8, sc


def xsums32(x, order=AMD64):
    x = _f32(x)
    out = np.empty(x.size // 32, np.float32)
    lib().ref_xsums32(_p(x), _p(out), out.size, order)
    return out


def xsums16(x, order=AMD64, scale32=True):
    x = _f32(x)
    out = np.empty(x.size // 16, np.float32)
    lib().ref_xsums16(_p(x), _p(out), out.size, order, int(scale32))
    return out


def row_bytes(qtype, cols):
    return int(lib().ref_row_bytes(qtype, cols))


# ---- row dots / matvec -----------------------------------------------------
def row_dot(qtype, row, q8, xscale, xsums, order=AMD64):
    row, q8 = _u8(row), np.ascontiguousarray(q8, np.int8)
    xscale = _f32(xscale)
    blocks = xscale.size
    L = lib()
    if qtype == Q4_K:
        return L.ref_q4k_dot(_p(row), _p(q8), _p(xscale), _p(_f32(xsums)), blocks, order)
    if qtype == Q6_K:
        return L.ref_q6k_dot(_p(row), _p(q8), _p(xscale), _p(_f32(xsums)), blocks, order)
    if qtype == Q8_0:
        return L.ref_q8_0_dot(_p(row), _p(q8), _p(xscale), blocks, order)
    xs = _f32(xsums if xsums is not None else np.zeros(1, np.float32))
    return L.ref_row_dot_any(qtype, _p(row), _p(q8), _p(xscale), _p(xs), blocks, order)


def row_dot_avx2(qtype, row, q8, xscale, xsums):
    row, q8 = _u8(row), np.ascontiguousarray(q8, np.int8)
    xscale = _f32(xscale)
    blocks = xscale.size
    L = lib()
    if qtype == Q4_K:
        return L.ref_q4k_dot_avx2(_p(row), _p(q8), _p(xscale), _p(_f32(xsums)), blocks)
    if qtype == Q6_K:
        return L.ref_q6k_dot_avx2(_p(row), _p(q8), _p(xscale), _p(_f32(xsums)), blocks)
    return L.ref_q8_0_dot_avx2(_p(row), _p(q8), _p(xscale), blocks)


def lane_ints(qtype, row, q8):
    row, q8 = _u8(row), np.ascontiguousarray(q8, np.int8)
    blocks = q8.size // 256
    out = np.empty(blocks * 8, np.int32)
    lib().ref_lane_ints(qtype, _p(row), _p(q8), blocks, _p(out))
    return out.reshape(blocks, 8)


def matvec(qtype, data, x, rows, cols, order=AMD64, threads=0):
    data, x = _u8(data), _f32(x)
    out = np.empty(rows, np.float32)
    rc = lib().ref_matvec(qtype, _p(data), _p(x), rows, cols, _p(out), order, threads)
    if rc != 0:
        raise ValueError("ref_matvec rejected the shape")
    return out


def matvec_batch(qtype, data, xs, rows, cols, order=AMD64, threads=0):
    data, xs = _u8(data), _f32(xs)
    p = xs.size // cols
    out = np.empty((p, rows), np.float32)
    rc = lib().ref_matvec_batch(qtype, _p(data), _p(xs), p, rows, cols, _p(out), order, threads)
    if rc != 0:
        raise ValueError("ref_matvec_batch rejected the shape")
    return out


def matvec_batch_fast(qtype, data, xs, rows, cols, threads=0):
    """AVX2 port (the timed CPU baseline); None if the host lacks AVX2."""
    data, xs = _u8(data), _f32(xs)
    p = xs.size // cols
    out = np.empty((p, rows), np.float32)
    rc = lib().ref_matvec_batch_fast(qtype, _p(data), _p(xs), p, rows, cols, _p(out), threads)
    return None if rc != 0 else out


def argmax_matvec(qtype, data, x, rows, cols, order=AMD64, threads=0):
    data, x = _u8(data), _f32(x)
    return int(lib().ref_argmax_matvec(qtype, _p(data), _p(x), rows, cols, order, threads))


def argmax_finite(logits):
    logits = _f32(logits)
    return int(lib().ref_argmax_finite(_p(logits), logits.size))


def apply_repeat_penalty(logits, recent, penalty):
    """applyRepeatPenalty (sampling.go:136-153) on a copy of logits."""
    out = np.array(logits, np.float32, copy=True)
    rec = np.ascontiguousarray(recent, np.uint32)
    lib().ref_apply_repeat_penalty(_p(out), out.size, _p(rec), rec.size, np.float32(penalty))
    return out


def argmax_penalized(logits, recent, penalty):
    """SampleWithScratch's greedy branch (sampling.go:86-89): penalty, then
    argmaxFiniteToken."""
    return argmax_finite(apply_repeat_penalty(logits, recent, penalty))


# ---- RTN encoders / decoders ---------------------------------------------
def quantize_rows(qtype, w, threads=0):
    w = _f32(w)
    rows, cols = w.shape
    out = np.empty(rows * row_bytes(qtype, cols), np.uint8)
    lib().ref_quantize_rows(qtype, _p(w), rows, cols, _p(out), threads)
    return out


def float_dot_supported(qtype):
    return bool(lib().ref_float_dot_supported(qtype))


def float_dot(qtype, row, x, cols):
    """One row's float-activation dot of a same-type fused group
    (DotQ8_0F32 / DotQ4_0F32 / DotQ4_1F32 / DotQ2KF32 / DotQ3KF32 /
    DotMXFP4F32)."""
    row, x = _u8(row), _f32(x)
    return float(lib().ref_float_dot(qtype, _p(row), _p(x), cols))


def matvec_float(qtype, data, x, rows, cols, threads=0):
    data, x = _u8(data), _f32(x)
    out = np.empty(rows, np.float32)
    if lib().ref_matvec_float(qtype, _p(data), _p(x), rows, cols, _p(out), threads) != 0:
        raise ValueError(f"no float row dot for type {qtype}")
    return out


def dequant_row(qtype, row, cols):
    row = _u8(row)
    out = np.empty(cols, np.float32)
    lib().ref_dequant_row(qtype, _p(row), cols, _p(out))
    return out


def dequant(qtype, data, rows, cols):
    data = _u8(data)
    rb = row_bytes(qtype, cols)
    return np.stack([dequant_row(qtype, data[r * rb:(r + 1) * rb], cols) for r in range(rows)])


# ---- vector helpers --------------------------------------------------------
def dot_f32(a, b):
    a, b = _f32(a), _f32(b)
    return lib().ref_dot_f32(_p(a), _p(b), min(a.size, b.size))


def dot_f32_f16(a, b):
    a, b = _f32(a), np.ascontiguousarray(b, np.uint16)
    return lib().ref_dot_f32_f16(_p(a), _p(b), min(a.size, b.size))


def has_avx2() -> bool:
    return bool(lib().ref_has_avx2())


def fast_exp(x):
    return lib().ref_fast_exp(float(x))


def silu_mul(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().ref_silu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().ref_rmsnorm(_p(x), _p(w), eps, x.size, _p(out))
    return out


def rope_inv_freq(theta, head_dim):
    out = np.empty(head_dim // 2, np.float32)
    lib().ref_rope_inv_freq(theta, head_dim, _p(out))
    return out


def rope_sincos(pos, inv):
    inv = _f32(inv)
    s = np.empty(inv.size, np.float32)
    c = np.empty(inv.size, np.float32)
    lib().ref_rope_sincos(pos, _p(inv), inv.size, _p(s), _p(c))
    return s, c


def rope_apply(vec, head_dim, n_heads, sinv, cosv):
    vec = _f32(vec).copy()
    sinv, cosv = _f32(sinv), _f32(cosv)
    lib().ref_rope_apply(_p(vec), head_dim, n_heads, sinv.size, _p(sinv), _p(cosv))
    return vec


def attend_group_f16(q, keys, values, q_heads, kstride, vstride, hd, vd, start, end, scale):
    """keys/values: uint16 arrays whose element 0 is the kv head's position-0 row."""
    q = _f32(q)
    keys = np.ascontiguousarray(keys, np.uint16)
    values = np.ascontiguousarray(values, np.uint16)
    out = np.zeros(q_heads * vd, np.float32)
    lib().ref_attend_group_f16(_p(q), _p(keys), _p(values), q_heads, kstride, vstride, hd, vd,
                               start, end, scale, _p(out))
    return out


# ---- llama decoder ---------------------------------------------------------
class _RefLlama(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "dim", "hidden", "n_heads", "n_kv_heads",
                                        "head_dim", "vocab", "max_len")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("emb_type", C.c_int), ("out_type", C.c_int),
        ("tok_embd", C.c_void_p), ("output", C.c_void_p), ("out_norm", C.c_void_p),
        ("layer_type", C.c_int),
    ] + [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3",
                                    "attn_norm", "ffn_norm", "types")] + [
        ("attn_scale", C.c_float)]


class Llama:
    """Owns a ref_llama_state over a model dict produced by the tests' model
    builder (numpy arrays kept alive here)."""

    def __init__(self, model, max_len, threads=0, fast=False):
        cfg = model["config"]
        self._keep = []
        L = lib()
        n = cfg["n_layers"]

        def ptr_array(arrs):
            arrs = [np.ascontiguousarray(a) for a in arrs]
            self._keep.extend(arrs)
            tab = (C.c_void_p * n)(*[a.ctypes.data for a in arrs])
            self._keep.append(tab)
            return C.cast(tab, C.c_void_p)

        s = _RefLlama()
        for k in ("n_layers", "dim", "hidden", "n_heads", "n_kv_heads", "head_dim", "vocab"):
            setattr(s, k, cfg[k])
        s.max_len = max_len
        s.rms_eps = cfg["rms_eps"]
        s.rope_theta = cfg["rope_theta"]
        s.attn_scale = cfg.get("attn_scale", 0.0)
        s.emb_type, s.out_type, s.layer_type = cfg["emb_type"], cfg["out_type"], cfg["layer_type"]
        for k in ("tok_embd", "output", "out_norm"):
            a = np.ascontiguousarray(model[k])
            self._keep.append(a)
            setattr(s, k, a.ctypes.data)
        for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "attn_norm", "ffn_norm"):
            setattr(s, k, ptr_array(model[k]))
        if "types" in model:  # per-matrix types, [n_layers][7] (wq wk wv wo w1 w2 w3)
            t = np.ascontiguousarray(np.asarray(model["types"], np.int32).reshape(n * 7))
            self._keep.append(t)
            s.types = t.ctypes.data
        self._s = s
        self.cfg = cfg
        self.state = L.ref_llama_state_new(C.byref(s), threads)
        # fast: row dots through the AVX2 port (bit-identical, for full-size models)
        L.ref_llama_set_fast(self.state, 1 if fast else 0)

    def close(self):
        if self.state:
            lib().ref_llama_state_free(self.state)
            self.state = None

    __del__ = close

    def set_repeat_penalty(self, penalty, window=64):
        """Repeat penalty over the last `window` tokens the state has seen
        (runtime.go repeatPenaltyWindow = 64); clears the window."""
        lib().ref_llama_set_repeat_penalty(self.state, np.float32(penalty), window)

    def decode(self, token, pos):
        hid = np.empty(self.cfg["dim"], np.float32)
        tok = lib().ref_llama_decode(self.state, token, pos, _p(hid))
        return int(tok), hid

    def prefill(self, tokens, start_pos=0, chunk=32):
        tokens = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        tok = lib().ref_llama_prefill(self.state, _p(tokens), tokens.size, start_pos, chunk,
                                      _p(logits))
        return int(tok), logits

    def generate(self, prompt, n_gen, chunk=32):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_gen, np.uint32)
        lib().ref_llama_generate(self.state, _p(prompt), prompt.size, n_gen, chunk, _p(out))
        return out

    def kcache(self, layer, max_len):
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        ptr = lib().ref_llama_kcache(self.state, layer)
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint16)), (max_len, kvd)).copy()

    def set_kv(self, layer, pos0, k16, v16):
        """Write f16 K/V rows (bit arrays [n][kv_dim]) into the state's cache at
        positions pos0.. (for starting a decode from another engine's prefill)."""
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        for get, rows in ((lib().ref_llama_kcache, k16), (lib().ref_llama_vcache, v16)):
            rows = np.ascontiguousarray(rows, np.uint16)
            assert rows.ndim == 2 and rows.shape[1] == kvd
            assert 0 <= pos0 and pos0 + rows.shape[0] <= self._s.max_len
            base = get(self.state, layer)
            C.memmove(base + 2 * pos0 * kvd, rows.ctypes.data, rows.nbytes)

    def vcache(self, layer, max_len):
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        ptr = lib().ref_llama_vcache(self.state, layer)
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint16)), (max_len, kvd)).copy()
