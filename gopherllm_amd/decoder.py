"""Resident llama decoder over the C ABI (gllm_hip_model_*): the device-side
counterpart of the reference's ForwardBodyInto / ForwardBatchInto and the
greedy loop of Runner.GenerateChatStreamUntil (runtime.go:1129-1170).

Weights are GGUF-layout bytes (host numpy arrays or device tensors); the
decoder borrows Weight handles, which it keeps alive.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import ModelConfig, call, call_ptr, load
from .api import KVCacheF16, Weight

LAYER_SLOTS = {"wq": _lib.T_WQ, "wk": _lib.T_WK, "wv": _lib.T_WV, "wo": _lib.T_WO,
               "w1": _lib.T_W1, "w2": _lib.T_W2, "w3": _lib.T_W3}


class LlamaDecoder:
    def __init__(self, config: dict, max_len: int):
        self.config = dict(config)
        c = ModelConfig()
        for k in ("n_layers", "dim", "hidden", "n_heads", "n_kv_heads", "head_dim", "vocab"):
            setattr(c, k, int(config[k]))
        c.max_len = int(max_len)
        c.rms_eps = float(config.get("rms_eps", 1e-5))
        c.rope_theta = float(config.get("rope_theta", 500000.0))
        self.max_len = max_len
        self._cfg = c
        self.handle = call_ptr("gllm_hip_model_new", C.byref(c))
        self._weights = []
        self._by_slot = {}  # (layer, slot) -> Weight
        self._norms = {}    # (layer, slot) -> host copy

    def release(self):
        if self.handle:
            load().gllm_hip_model_release(self.handle)
            self.handle = None
        for w in self._weights:
            w.release()
        self._weights = []

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def set_weight(self, layer: int, slot: int, w: Weight):
        call("gllm_hip_model_set_weight", self.handle, layer, slot, w.handle)
        self._weights.append(w)
        self._by_slot[(layer, slot)] = w

    def set_norm(self, layer: int, slot: int, values):
        v = np.ascontiguousarray(values, np.float32)
        call("gllm_hip_model_set_norm", self.handle, layer, slot, v.ctypes.data_as(C.c_void_p))
        self._norms[(layer, slot)] = v.copy()

    def weights_by_slot(self):
        """{(layer, slot): Weight}; the embedding and output sit at layer 0."""
        return dict(self._by_slot)

    def norm(self, layer: int, slot: int):
        return self._norms[(layer, slot)]

    @classmethod
    def from_gguf(cls, source, max_len: int = 0) -> "LlamaDecoder":
        """LoadModel (model.go:1872-1930) for a llama GGUF: source is a path
        or a gguf.GGUFFile.  The weights are read from the file mapping and
        owned by the model; max_len <= 0 takes llama.context_length."""
        from .gguf import GGUFFile
        f = source if isinstance(source, GGUFFile) else GGUFFile(source)
        h = call_ptr("gllm_hip_model_from_gguf", f.handle, int(max_len))
        d = cls.__new__(cls)
        arch = "llama."
        d.config = {
            "n_layers": f.get_u32(arch + "block_count"), "dim": f.get_u32(arch + "embedding_length"),
            "hidden": f.get_u32(arch + "feed_forward_length"),
            "n_heads": f.get_u32(arch + "attention.head_count"),
            "n_kv_heads": f.get_u32(arch + "attention.head_count_kv"),
            "vocab": f.tensors()[f.find("token_embd.weight")].dims[1],
        }
        d.config["head_dim"] = d.config["dim"] // d.config["n_heads"]
        d.max_len = max_len if max_len > 0 else f.get_u32(arch + "context_length")
        d._cfg = None
        d.handle = h
        d._weights, d._by_slot, d._norms = [], {}, {}
        if f is not source:
            f.close()  # the model holds device copies; the mapping can go
        return d

    @classmethod
    def from_host_model(cls, model: dict, max_len: int) -> "LlamaDecoder":
        """model: {"config", "tok_embd", "output", "out_norm", "wq".."w3" lists,
        "attn_norm"/"ffn_norm" lists, optional "types" [n_layers][7] in wq wk
        wv wo w1 w2 w3 order} with GGUF-layout bytes."""
        cfg = model["config"]
        d = cls(cfg, max_len)
        dim, hidden = cfg["dim"], cfg["hidden"]
        qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
        shapes = {"wq": (qd, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, qd),
                  "w1": (hidden, dim), "w2": (dim, hidden), "w3": (hidden, dim)}
        lt = cfg["layer_type"]
        d.set_weight(0, _lib.T_TOK_EMBD, Weight.from_host(model["tok_embd"], cfg["emb_type"],
                                                          cfg["vocab"], dim))
        d.set_weight(0, _lib.T_OUTPUT, Weight.from_host(model["output"], cfg["out_type"],
                                                        cfg["vocab"], dim))
        d.set_norm(0, _lib.T_OUT_NORM, model["out_norm"])
        types = model.get("types")  # optional [n_layers][7], wq wk wv wo w1 w2 w3
        order = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")
        for l in range(cfg["n_layers"]):
            for k, slot in LAYER_SLOTS.items():
                r, c = shapes[k]
                t = types[l][order.index(k)] if types is not None else lt
                d.set_weight(l, slot, Weight.from_host(model[k][l], t, r, c))
            d.set_norm(l, _lib.T_ATTN_NORM, model["attn_norm"][l])
            d.set_norm(l, _lib.T_FFN_NORM, model["ffn_norm"][l])
        return d

    # ---------------------------------------------------------------- steps
    def decode(self, token: int, pos: int) -> int:
        nxt = C.c_uint32(0)
        call("gllm_hip_model_decode", self.handle, int(token), int(pos), C.byref(nxt))
        return int(nxt.value)

    def prefill(self, tokens, start_pos: int = 0, want_logits: bool = False):
        t = np.ascontiguousarray(tokens, np.uint32)
        first = C.c_uint32(0)
        logits = np.empty(self.config["vocab"], np.float32) if want_logits else None
        call("gllm_hip_model_prefill", self.handle, t.ctypes.data_as(C.c_void_p), t.size,
             start_pos, C.byref(first),
             logits.ctypes.data_as(C.c_void_p) if logits is not None else None)
        return (int(first.value), logits) if want_logits else int(first.value)

    def set_repeat_penalty(self, penalty: float, window: int = 64):
        """Repeat penalty on every greedy choice, over the last `window`
        tokens given to prefill / decode (runtime.go repeatPenaltyWindow = 64,
        forwardGreedyToken runtime.go:1607).  Clears the window."""
        call("gllm_hip_model_set_repeat_penalty", self.handle, float(penalty), int(window))

    def hidden(self):
        out = np.empty(self.config["dim"], np.float32)
        call("gllm_hip_model_hidden", self.handle, out.ctypes.data_as(C.c_void_p))
        return out

    def kv_cache(self) -> KVCacheF16:
        h = load().gllm_hip_model_kv(self.handle)
        kvd = self.config["n_kv_heads"] * self.config["head_dim"]
        return KVCacheF16(self.config["n_layers"], kvd, kvd, self.max_len, handle=h, owned=False)

    def generate(self, prompt, n_gen: int):
        """Greedy: first token from the prefill logits, then one decode step
        per further token (runtime.go:1129-1170)."""
        if n_gen <= 0:
            return np.zeros(0, np.uint32)
        out = np.empty(n_gen, np.uint32)
        tok = self.prefill(prompt)
        out[0] = tok
        n = len(prompt)
        for i in range(1, n_gen):
            tok = self.decode(tok, n + i - 1)
            out[i] = tok
        return out
