"""GGUF files: a streaming writer (NewGGUFWriter, gguf_write.go:309-442) and a
handle over the native reader in libgllm_hip.so (ParseGGUF gguf.go:493-568 on
a read-only mapping, mmap.go:11-14), with the uploads that turn a file into
device weights (loadWeight model.go:2357-2476) and a resident llama decoder
(LoadModel model.go:1872-1930).

The writer builds the synthetic models as files; the reader is the product's
load path.  Parsing needs no GPU; uploading does.
"""
from __future__ import annotations

import ctypes as C
import struct
from typing import NamedTuple

import numpy as np

from ._lib import GllmError, call, call_ptr, last_error, load

# GGUF metadata wire kinds (cursor.value, gguf.go:671-767)
KINDS = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7,
         "str": 8, "array": 9, "u64": 10, "i64": 11, "f64": 12}
_KIND_NAME = {v: k for k, v in KINDS.items()}
_SCALAR_FMT = {"u8": "<B", "i8": "<b", "u16": "<H", "i16": "<h", "u32": "<I", "i32": "<i",
               "f32": "<f", "u64": "<Q", "i64": "<q", "f64": "<d"}
_NP_KIND = {np.dtype(np.uint8): "u8", np.dtype(np.int8): "i8", np.dtype(np.uint16): "u16",
            np.dtype(np.int16): "i16", np.dtype(np.uint32): "u32", np.dtype(np.int32): "i32",
            np.dtype(np.float32): "f32", np.dtype(np.uint64): "u64", np.dtype(np.int64): "i64",
            np.dtype(np.float64): "f64", np.dtype(np.bool_): "bool"}


class MetaValue(NamedTuple):
    """One metadata value: kind is a KINDS name.  An "array" value is a list
    of str (a str array), a list of bool, a numpy array (its dtype names the
    element kind) or a list of MetaValue of one kind (possibly arrays)."""
    kind: str
    value: object


class PlannedTensor(NamedTuple):
    name: str
    dims: tuple          # GGUF order: dims[0] varies fastest (cols of a matrix)
    dtype: int           # ggml type id


def data_size(dtype: int, n: int) -> int:
    """GGMLType.DataSize (gguf.go:241-297), from the library; 0 if unsized."""
    return int(load().gllm_hip_ggml_data_size(int(dtype), int(n)))


def _align_up(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def _payload(kind: str, value) -> bytes:
    """Value bytes without the kind tag (writeMetaValuePayload)."""
    if kind in _SCALAR_FMT:
        return struct.pack(_SCALAR_FMT[kind], value)
    if kind == "bool":
        return struct.pack("<B", 1 if value else 0)
    if kind == "str":
        b = value.encode() if isinstance(value, str) else bytes(value)
        return struct.pack("<Q", len(b)) + b
    if kind == "array":
        return _array_payload(value)
    raise ValueError(f"unknown metadata kind {kind!r}")


def _array_payload(value) -> bytes:
    """writeMetaArray (gguf_write.go:203-285): element tag, count, payloads."""
    if isinstance(value, np.ndarray):
        kind = _NP_KIND.get(value.dtype)
        if kind is None:
            raise ValueError(f"unsupported array dtype {value.dtype}")
        body = value.astype(np.uint8 if kind == "bool" else value.dtype.newbyteorder("<"),
                            copy=False).tobytes()
        return struct.pack("<IQ", KINDS[kind], value.size) + body
    items = list(value)
    if items and all(isinstance(x, MetaValue) for x in items):
        kind = items[0].kind
        if any(x.kind != kind for x in items):
            raise ValueError("GGUF arrays are homogeneous")
        return struct.pack("<IQ", KINDS[kind], len(items)) + b"".join(
            _payload(kind, x.value) for x in items)
    if not items:  # a declared element type is still required; u8, as the reference
        return struct.pack("<IQ", KINDS["u8"], 0)
    if all(isinstance(x, str) for x in items):
        return struct.pack("<IQ", KINDS["str"], len(items)) + b"".join(_payload("str", x) for x in items)
    if all(isinstance(x, bool) for x in items):
        return struct.pack("<IQ", KINDS["bool"], len(items)) + bytes(1 if x else 0 for x in items)
    raise ValueError("array values: list of str / bool / MetaValue, or a numpy array")


class GGUFWriter:
    """NewGGUFWriter / WriteTensor / Close (gguf_write.go:309-442): header
    (version 3), metadata with general.alignment set to the padding used,
    the tensor table with offsets planned from DataSize, then each tensor's
    bytes in plan order, padded to the next aligned offset."""

    def __init__(self, f, metadata: dict, planned, alignment: int = 32):
        if alignment <= 0:
            alignment = 32
        meta = dict(metadata)
        meta["general.alignment"] = MetaValue("u32", alignment)
        self.f, self.alignment = f, alignment
        self.pos = 0
        self._write(b"GGUF" + struct.pack("<IQQ", 3, len(planned), len(meta)))
        for key, v in meta.items():
            if v.kind not in KINDS:
                raise ValueError(f"metadata {key!r}: unknown kind {v.kind!r}")
            self._write(_payload("str", key) + struct.pack("<I", KINDS[v.kind]) + _payload(v.kind, v.value))
        self.tensors = []
        off = 0
        for p in planned:
            n = int(np.prod(p.dims, dtype=np.int64)) if len(p.dims) else 1
            size = data_size(p.dtype, n)
            if size == 0 and n:
                raise ValueError(f"tensor {p.name!r}: unsupported output type {p.dtype}")
            self.tensors.append((p, off, size))
            off = _align_up(off + size, alignment)
        for p, o, _ in self.tensors:
            self._write(_payload("str", p.name) + struct.pack("<I", len(p.dims)) +
                        b"".join(struct.pack("<Q", int(d)) for d in p.dims) + struct.pack("<IQ", p.dtype, o))
        self._write(bytes(_align_up(self.pos, alignment) - self.pos))
        self.data_offset = self.pos
        self.next = 0

    def _write(self, b: bytes):
        self.f.write(b)
        self.pos += len(b)

    def write_tensor(self, data):
        if self.next >= len(self.tensors):
            raise ValueError(f"write_tensor called more times than planned ({len(self.tensors)} tensors)")
        p, _, size = self.tensors[self.next]
        b = memoryview(np.ascontiguousarray(data)).cast("B")
        if len(b) != size:
            raise ValueError(f"tensor {p.name!r}: got {len(b)} bytes, want {size}")
        self._write(b)
        self.next += 1
        if self.next < len(self.tensors):
            want = self.data_offset + self.tensors[self.next][1]
            self._write(bytes(want - self.pos))

    def close(self):
        if self.next != len(self.tensors):
            raise ValueError(f"GGUFWriter closed after {self.next} of {len(self.tensors)} planned tensors")
        self.f.flush()


class TensorInfo(NamedTuple):
    name: str
    dims: tuple
    dtype: int
    offset: int   # relative to the data offset
    nbytes: int


class GGUFFile:
    """A parsed GGUF file (native reader; the tensor bytes stay in the
    mapping).  Open from a path, or parse bytes held by this object."""

    def __init__(self, path=None, data: bytes | None = None):
        L = load()
        if (path is None) == (data is None):
            raise ValueError("give a path or data")
        if path is not None:
            self.handle = L.gllm_hip_gguf_open(str(path).encode())
        else:
            self._buf = C.create_string_buffer(bytes(data), len(data))
            self.handle = L.gllm_hip_gguf_parse(C.cast(self._buf, C.c_void_p), len(data))
        if not self.handle:
            raise GllmError("gllm_hip_gguf_open", -1, last_error())

    def close(self):
        if getattr(self, "handle", None):
            load().gllm_hip_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def version(self) -> int:
        return int(load().gllm_hip_gguf_version(self.handle))

    @property
    def data_offset(self) -> int:
        return int(load().gllm_hip_gguf_data_offset(self.handle))

    def metadata_keys(self):
        L = load()
        return [L.gllm_hip_gguf_metadata_key(self.handle, i).decode()
                for i in range(L.gllm_hip_gguf_n_metadata(self.handle))]

    def tensors(self):
        out = []
        for i in range(load().gllm_hip_gguf_n_tensors(self.handle)):
            name, nd, ty = C.c_char_p(), C.c_int(), C.c_int()
            dims = (C.c_uint64 * 8)()
            off, nb = C.c_uint64(), C.c_uint64()
            call("gllm_hip_gguf_tensor", self.handle, i, C.byref(name), C.byref(nd), dims,
                 C.byref(ty), C.byref(off), C.byref(nb))
            out.append(TensorInfo(name.value.decode(), tuple(int(dims[k]) for k in range(nd.value)),
                                  ty.value, off.value, nb.value))
        return out

    def find(self, name: str) -> int:
        return int(load().gllm_hip_gguf_find_tensor(self.handle, name.encode()))

    def tensor_bytes(self, name: str) -> bytes:
        """A copy of the tensor's bytes (as loadWeight borrows them)."""
        i = self.find(name)
        if i < 0:
            raise KeyError(name)
        info = self.tensors()[i]
        ptr = load().gllm_hip_gguf_tensor_data(self.handle, i)
        return C.string_at(ptr, info.nbytes)

    def kind(self, key: str):
        """(kind name, element kind name or None, count) of a metadata value."""
        k, e, n = C.c_int(), C.c_int(), C.c_uint64()
        call("gllm_hip_gguf_meta_kind", self.handle, key.encode(), C.byref(k), C.byref(e), C.byref(n))
        return _KIND_NAME[k.value], (_KIND_NAME.get(e.value) if e.value >= 0 else None), n.value

    def _get(self, fn, ctype, key, idx):
        out = ctype()
        call(fn, self.handle, key.encode(), idx, C.byref(out))
        return out.value

    def get_u32(self, key: str, idx: int = -1) -> int:
        """AsU32 (gguf.go:308): any integer kind, cast to 32 bits."""
        return self._get("gllm_hip_gguf_get_u32", C.c_uint32, key, idx)

    def get_u64(self, key: str, idx: int = -1) -> int:
        return self._get("gllm_hip_gguf_get_u64", C.c_uint64, key, idx)

    def get_f32(self, key: str, idx: int = -1) -> float:
        """AsF32 (gguf.go:331): f32 or f64, as float32."""
        return self._get("gllm_hip_gguf_get_f32", C.c_float, key, idx)

    def get_f64(self, key: str, idx: int = -1) -> float:
        return self._get("gllm_hip_gguf_get_f64", C.c_double, key, idx)

    def get_bool(self, key: str, idx: int = -1) -> bool:
        return bool(self._get("gllm_hip_gguf_get_bool", C.c_int, key, idx))

    def get_str(self, key: str, idx: int = -1) -> str:
        p, n = C.c_void_p(), C.c_size_t()
        call("gllm_hip_gguf_get_str", self.handle, key.encode(), idx, C.byref(p), C.byref(n))
        return C.string_at(p, n.value).decode()

    def load_weight(self, name: str):
        """loadWeight: the tensor as a device weight (rows = dims[1])."""
        from .api import Weight
        h = call_ptr("gllm_hip_gguf_load_weight", self.handle, name.encode())
        info = self.tensors()[self.find(name)]
        rows = info.dims[1] if len(info.dims) > 1 else 1
        return Weight(h, info.dtype, rows, info.dims[0])


def write_llama_gguf(path, model: dict, alignment: int = 32, name: str = "synthetic llama",
                     extra_meta: dict | None = None, extra_tensors=()):
    """Write a model dict of the tests' / benchmark's builder (GGUF-layout
    tensor bytes plus "config") as a llama GGUF file with llama.cpp's tensor
    names and hyperparameter keys (the layout ConfigFromGGUF / LoadModel
    read, model.go:328-420, 1872-2090).  extra_meta ({key: MetaValue})
    and extra_tensors ((name, dims, dtype, bytes) tuples) are added as given;
    a config "attn_scale" is written as llama.attention.scale."""
    cfg = model["config"]
    dim, hidden, nl = cfg["dim"], cfg["hidden"], cfg["n_layers"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    meta = {
        "general.architecture": MetaValue("str", "llama"),
        "general.name": MetaValue("str", name),
        "llama.block_count": MetaValue("u32", nl),
        "llama.context_length": MetaValue("u32", int(cfg.get("context_length", 8192))),
        "llama.embedding_length": MetaValue("u32", dim),
        "llama.feed_forward_length": MetaValue("u32", hidden),
        "llama.attention.head_count": MetaValue("u32", cfg["n_heads"]),
        "llama.attention.head_count_kv": MetaValue("u32", cfg["n_kv_heads"]),
        "llama.attention.key_length": MetaValue("u32", cfg["head_dim"]),
        "llama.attention.value_length": MetaValue("u32", cfg["head_dim"]),
        "llama.rope.freq_base": MetaValue("f32", float(cfg["rope_theta"])),
        "llama.attention.layer_norm_rms_epsilon": MetaValue("f32", float(cfg["rms_eps"])),
        "llama.vocab_size": MetaValue("u32", cfg["vocab"]),
    }
    if cfg.get("attn_scale"):
        meta["llama.attention.scale"] = MetaValue("f32", float(cfg["attn_scale"]))
    meta.update(extra_meta or {})
    F32 = 0
    planned, blobs = [], []

    def add(tname, dims, dtype, data):
        planned.append(PlannedTensor(tname, tuple(dims), dtype))
        blobs.append(data)

    add("token_embd.weight", (dim, cfg["vocab"]), cfg["emb_type"], model["tok_embd"])
    add("output_norm.weight", (dim,), F32, np.asarray(model["out_norm"], np.float32))
    if model.get("output") is not None:
        add("output.weight", (dim, cfg["vocab"]), cfg["out_type"], model["output"])
    shapes = {"attn_q": ("wq", qd, dim), "attn_k": ("wk", kvd, dim), "attn_v": ("wv", kvd, dim),
              "attn_output": ("wo", dim, qd), "ffn_gate": ("w1", hidden, dim),
              "ffn_down": ("w2", dim, hidden), "ffn_up": ("w3", hidden, dim)}
    types = model.get("types")  # optional [n_layers][7], wq wk wv wo w1 w2 w3 (mixed files)
    order = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")
    for l in range(nl):
        add(f"blk.{l}.attn_norm.weight", (dim,), F32, np.asarray(model["attn_norm"][l], np.float32))
        for tname, (key, rows, cols) in shapes.items():
            t = types[l][order.index(key)] if types is not None else cfg["layer_type"]
            add(f"blk.{l}.{tname}.weight", (cols, rows), t, model[key][l])
        add(f"blk.{l}.ffn_norm.weight", (dim,), F32, np.asarray(model["ffn_norm"][l], np.float32))
    for tname, dims, dtype, data in extra_tensors:
        add(tname, dims, dtype, data)
    with open(path, "wb") as f:
        w = GGUFWriter(f, meta, planned, alignment)
        for b in blobs:
            w.write_tensor(b)
        w.close()
    return path
