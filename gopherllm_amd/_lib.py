"""ctypes binding of libgllm_hip.so (the C ABI declared in include/gllm_hip.h).

The product path has exactly one implementation: the HIP library.  Loading
fails loudly when it has not been built; nothing here falls back to a CPU or
PyTorch computation.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgllm_hip.so")

TYPE_F32, TYPE_F16, TYPE_BF16, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 30, 8, 12, 14
TYPE_Q4_0, TYPE_Q4_1, TYPE_Q2_K, TYPE_Q3_K, TYPE_Q5_K, TYPE_MXFP4 = 2, 3, 10, 11, 13, 39
OK, EINVAL, EDEVICE, ENOMEM, EUNSUP = 0, -1, -2, -3, -4
ATTN_EXACT, ATTN_SPLITK = 0, 1
(T_WQ, T_WK, T_WV, T_WO, T_W1, T_W2, T_W3, T_TOK_EMBD, T_OUTPUT, T_ATTN_NORM, T_FFN_NORM,
 T_OUT_NORM) = range(12)


class GllmError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "dim", "hidden", "n_heads", "n_kv_heads",
                                        "head_dim", "vocab", "max_len")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float)]


vp, i32, u32, u64, f32, sz = C.c_void_p, C.c_int, C.c_uint32, C.c_uint64, C.c_float, C.c_size_t

# name -> (restype, argtypes); int-returning calls are error-checked.
SIGNATURES = {
    "gllm_hip_available": (i32, []),
    "gllm_hip_last_error": (C.c_char_p, []),
    "gllm_hip_set_device": (i32, [i32]),
    "gllm_hip_version": (C.c_char_p, []),
    "gllm_hip_stream_release": (i32, [vp]),
    "gllm_hip_weight_new": (vp, [vp, sz, i32, i32, i32]),
    "gllm_hip_weight_from_device": (vp, [vp, sz, i32, i32, i32, vp]),
    "gllm_hip_weight_release": (None, [vp]),
    "gllm_hip_weight_shape": (i32, [vp, vp, vp, vp]),
    "gllm_hip_weight_download_dev": (i32, [vp, vp, vp]),
    "gllm_hip_weight_rows_dev": (i32, [vp, vp, i32, vp, vp]),
    "gllm_hip_matvec": (i32, [vp, vp, vp]),
    "gllm_hip_matvec2": (i32, [vp, vp, vp, vp, vp]),
    "gllm_hip_matvec3": (i32, [vp, vp, vp, vp, vp, vp, vp]),
    "gllm_hip_matvec_batch": (i32, [vp, vp, i32, vp]),
    "gllm_hip_argmax": (i32, [vp, vp, vp]),
    "gllm_hip_argmax_penalized": (i32, [vp, vp, vp, i32, f32, vp]),
    "gllm_hip_argmax_penalized_dev": (i32, [vp, vp, vp, i32, f32, vp, vp]),
    "gllm_hip_matvec_dev": (i32, [vp, vp, i32, vp, i32, vp]),
    "gllm_hip_matvec_dev_noalloc": (i32, [vp, vp, i32, vp, i32, vp]),
    "gllm_hip_matvec_multi_dev": (i32, [i32, vp, vp, i32, vp, vp, vp]),
    "gllm_hip_swiglu_down_dev": (i32, [vp, vp, vp, vp, vp, vp]),
    "gllm_hip_argmax_dev": (i32, [vp, vp, vp, vp]),
    "gllm_hip_act_bytes": (sz, [i32, i32]),
    "gllm_hip_q8k_prepare_dev": (i32, [vp, i32, i32, vp, vp]),
    "gllm_hip_matvec_q8_dev": (i32, [vp, vp, i32, vp, i32, vp]),
    "gllm_hip_q8k_quantize_dev": (i32, [vp, i32, i32, vp, vp, vp]),
    "gllm_hip_lane_ints_dev": (i32, [vp, vp, vp, vp]),
    "gllm_hip_quantize_rows_dev": (i32, [i32, vp, i32, i32, vp, vp]),
    "gllm_hip_fill_normal_dev": (i32, [vp, sz, u64, f32, vp]),
    "gllm_hip_kv_new": (vp, [i32, i32, i32, i32]),
    "gllm_hip_kv_release": (None, [vp]),
    "gllm_hip_kv_k_dev": (vp, [vp, i32]),
    "gllm_hip_kv_v_dev": (vp, [vp, i32]),
    "gllm_hip_kv_read": (i32, [vp, i32, i32, i32, vp, vp]),
    "gllm_hip_kv_store": (i32, [vp, i32, i32, vp, vp]),
    "gllm_hip_kv_store_dev": (i32, [vp, i32, i32, vp, vp, vp]),
    "gllm_hip_attend_group": (i32, [vp, i32, i32, vp, i32, i32, i32, i32, i32, f32, f32, vp]),
    "gllm_hip_attend_dev": (i32, [vp, i32, vp, i32, i32, i32, i32, i32, f32, i32, vp, vp]),
    "gllm_hip_model_new": (vp, [vp]),
    "gllm_hip_model_release": (None, [vp]),
    "gllm_hip_model_set_weight": (i32, [vp, i32, i32, vp]),
    "gllm_hip_model_set_norm": (i32, [vp, i32, i32, vp]),
    "gllm_hip_model_decode": (i32, [vp, u32, i32, vp]),
    "gllm_hip_model_prefill": (i32, [vp, vp, i32, i32, vp, vp]),
    "gllm_hip_model_hidden": (i32, [vp, vp]),
    "gllm_hip_model_set_repeat_penalty": (i32, [vp, f32, i32]),
    "gllm_hip_gguf_open": (vp, [C.c_char_p]),
    "gllm_hip_gguf_parse": (vp, [vp, sz]),
    "gllm_hip_gguf_close": (None, [vp]),
    "gllm_hip_gguf_version": (u32, [vp]),
    "gllm_hip_gguf_data_offset": (sz, [vp]),
    "gllm_hip_gguf_n_tensors": (i32, [vp]),
    "gllm_hip_gguf_n_metadata": (i32, [vp]),
    "gllm_hip_gguf_metadata_key": (C.c_char_p, [vp, i32]),
    "gllm_hip_gguf_tensor": (i32, [vp, i32, vp, vp, vp, vp, vp, vp]),
    "gllm_hip_gguf_find_tensor": (i32, [vp, C.c_char_p]),
    "gllm_hip_gguf_tensor_data": (vp, [vp, i32]),
    "gllm_hip_gguf_meta_kind": (i32, [vp, C.c_char_p, vp, vp, vp]),
    "gllm_hip_gguf_get_u32": (i32, [vp, C.c_char_p, i32, vp]),
    "gllm_hip_gguf_get_u64": (i32, [vp, C.c_char_p, i32, vp]),
    "gllm_hip_gguf_get_f32": (i32, [vp, C.c_char_p, i32, vp]),
    "gllm_hip_gguf_get_f64": (i32, [vp, C.c_char_p, i32, vp]),
    "gllm_hip_gguf_get_bool": (i32, [vp, C.c_char_p, i32, vp]),
    "gllm_hip_gguf_get_str": (i32, [vp, C.c_char_p, i32, vp, vp]),
    "gllm_hip_ggml_data_size": (u64, [i32, u64]),
    "gllm_hip_gguf_load_weight": (vp, [vp, C.c_char_p]),
    "gllm_hip_model_from_gguf": (vp, [vp, i32]),
    "gllm_hip_model_kv": (vp, [vp]),
}

_lib = None


def lib_path() -> str:
    return LIB_PATH


def load():
    """Load libgllm_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m gopherllm_amd.build` "
                           "(or __graft_entry__.build()); there is no fallback implementation")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    msg = load().gllm_hip_last_error()
    return msg.decode() if msg else ""


def call(name, *args):
    """Call an int-returning entry point; raise GllmError on failure."""
    rc = getattr(load(), name)(*args)
    if rc != OK:
        raise GllmError(name, rc, last_error())
    return rc


def call_ptr(name, *args):
    """Call a handle-returning entry point; raise GllmError on NULL."""
    p = getattr(load(), name)(*args)
    if not p:
        raise GllmError(name, 0, last_error())
    return p
