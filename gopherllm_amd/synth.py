"""Synthetic llama-shaped models built directly in HBM.

The benchmark configuration names a Llama-3-8B-shaped decoder with random
weights: every attention / FFN matrix drawn N(0, 0.02) and encoded Q4_K with
the reference's RTN encoder (QuantizeRowQ4K, quantize_rtn.go:128), the output
head encoded Q6_K (QuantizeRowQ6K, quantize_rtn.go:331), RMSNorm weights 1.0.
Tensors are generated on the device (gllm_hip_fill_normal_dev, a counter-based
generator keyed by (seed, tensor)) and encoded there
(gllm_hip_quantize_rows_dev), so a 4.4 GB model is resident in about a
second.  `host_model` downloads the GGUF-layout bytes (undoing the upload
repack) for host-side checking.
"""
from __future__ import annotations

import numpy as np

from . import _lib
from .api import Weight, fill_normal_dev, quantize_rows_dev, row_bytes
from .decoder import LAYER_SLOTS, LlamaDecoder

# Llama-3-8B shape; token_embd is Q4_K (one row read
# per token), output Q6_K.
LLAMA3_8B = dict(n_layers=32, dim=4096, hidden=14336, n_heads=32, n_kv_heads=8, head_dim=128,
                 vocab=128256, rms_eps=1e-5, rope_theta=500000.0, emb_type=_lib.TYPE_Q4_K,
                 out_type=_lib.TYPE_Q6_K, layer_type=_lib.TYPE_Q4_K)

SLOT_IDS = {"wq": 0, "wk": 1, "wv": 2, "wo": 3, "w1": 4, "w2": 5, "w3": 6, "tok_embd": 7,
            "output": 8}


def tensor_seed(seed: int, layer: int, name: str) -> int:
    """Generator key of one tensor: distinct for every (seed, layer, tensor)."""
    return (int(seed) * 1_000_003 + (layer + 1) * 101 + SLOT_IDS[name]) & 0x7FFFFFFFFFFFFFFF


def layer_shapes(cfg):
    dim, hidden = cfg["dim"], cfg["hidden"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    return {"wq": (qd, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, qd),
            "w1": (hidden, dim), "w2": (dim, hidden), "w3": (hidden, dim)}


class _Scratch:
    """Reused f32 / byte device buffers for generating one tensor at a time."""

    def __init__(self, torch, max_elems, max_bytes):
        self.f = torch.empty(max_elems, dtype=torch.float32, device="cuda")
        self.b = torch.empty(max_bytes, dtype=torch.uint8, device="cuda")

    def weight(self, qtype, rows, cols, key, std=0.02) -> Weight:
        n = rows * cols
        src = self.f[:n].view(rows, cols)
        fill_normal_dev(src, key, std)
        nbytes = rows * row_bytes(qtype, cols)
        dst = self.b[:nbytes]
        quantize_rows_dev(qtype, src, dst)
        return Weight.from_device(dst, qtype, rows, cols)


def q4km_type(cfg: dict, layer: int, name: str) -> int:
    """Q4_K_M-style mix (llama.cpp's Q4_K_M keeps attn_v and ffn_down at a
    higher precision on part of the layers): Q6_K for those two tensors on
    every other layer, the configuration's layer type elsewhere."""
    return _lib.TYPE_Q6_K if name in ("wv", "w2") and layer % 2 == 0 else cfg["layer_type"]


def build_decoder(cfg: dict, max_len: int, seed: int = 1, type_of=None) -> LlamaDecoder:
    """A resident decoder with synthetic weights of shape `cfg`; type_of(cfg,
    layer, name) picks a layer tensor's type (default: cfg["layer_type"])."""
    import torch

    shapes = layer_shapes(cfg)
    tof = type_of or (lambda c, l, name: c["layer_type"])
    types = {tof(cfg, l, name) for l in range(cfg["n_layers"]) for name in shapes}
    big = max([r * c for r, c in shapes.values()] + [cfg["vocab"] * cfg["dim"]])
    big_bytes = max([r * row_bytes(t, c) for r, c in shapes.values() for t in types] +
                    [cfg["vocab"] * row_bytes(t, cfg["dim"]) for t in (cfg["emb_type"], cfg["out_type"])])
    sc = _Scratch(torch, big, big_bytes)
    d = LlamaDecoder(cfg, max_len)
    d.set_weight(0, _lib.T_TOK_EMBD,
                 sc.weight(cfg["emb_type"], cfg["vocab"], cfg["dim"], tensor_seed(seed, -1, "tok_embd")))
    d.set_weight(0, _lib.T_OUTPUT,
                 sc.weight(cfg["out_type"], cfg["vocab"], cfg["dim"], tensor_seed(seed, -1, "output")))
    ones = np.ones(cfg["dim"], np.float32)
    d.set_norm(0, _lib.T_OUT_NORM, ones)
    for l in range(cfg["n_layers"]):
        for name, slot in LAYER_SLOTS.items():
            r, c = shapes[name]
            d.set_weight(l, slot, sc.weight(tof(cfg, l, name), r, c, tensor_seed(seed, l, name)))
        d.set_norm(l, _lib.T_ATTN_NORM, ones)
        d.set_norm(l, _lib.T_FFN_NORM, ones)
    torch.cuda.synchronize()
    del sc
    return d


def host_model(d: LlamaDecoder) -> dict:
    """GGUF-layout host copies of a decoder's weights, in the model-dict form
    the tests' builders produce (for host-side checking)."""
    import torch

    cfg = dict(d.config)
    by_slot = {}
    for (layer, slot), w in d.weights_by_slot().items():
        buf = torch.empty(w.rows * row_bytes(w.type, w.cols), dtype=torch.uint8, device="cuda")
        w.download_dev(buf)
        torch.cuda.synchronize()
        by_slot[(layer, slot)] = buf.cpu().numpy()
        del buf
    m = {"config": cfg, "tok_embd": by_slot[(0, _lib.T_TOK_EMBD)],
         "output": by_slot[(0, _lib.T_OUTPUT)], "out_norm": d.norm(0, _lib.T_OUT_NORM)}
    for name, slot in LAYER_SLOTS.items():
        m[name] = [by_slot[(l, slot)] for l in range(cfg["n_layers"])]
    m["attn_norm"] = [d.norm(l, _lib.T_ATTN_NORM) for l in range(cfg["n_layers"])]
    m["ffn_norm"] = [d.norm(l, _lib.T_FFN_NORM) for l in range(cfg["n_layers"])]
    return m
