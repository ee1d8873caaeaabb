"""gopherllm_amd -- MI355X (gfx950) HIP implementation of GopherLLM's
quantized matvec (Q4_K / Q6_K / Q8_0 x Q8K) and F16-KV GQA decode-attention
hot path, behind the C ABI of include/gllm_hip.h.

The Python layer only binds that ABI (ctypes); all arithmetic runs in
libgllm_hip.so.
"""
from ._lib import (TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q2_K,  # noqa: F401
                   TYPE_F32, TYPE_F16, TYPE_BF16, TYPE_Q3_K, TYPE_Q5_K, TYPE_MXFP4, ATTN_EXACT, ATTN_SPLITK, GllmError,
                   OK, EINVAL, EDEVICE, ENOMEM, EUNSUP, lib_path, load)
from .api import (KVCacheF16, Weight, act_bytes, available, q8k_prepare_dev, fill_normal_dev, matvec2_into,  # noqa: F401
                  matvec3_into, matvec_multi_dev, matvec_q4k_into, matvec_q6k_into,
                  matvec_q8_0_into, q8k_quantize_dev, quantize_rows_dev, row_bytes,
                  stream_release, swiglu_down_dev)

__all__ = [n for n in dir() if not n.startswith("_")]
