"""GGUF container: the native reader (ParseGGUF gguf.go:493-568) and the
writer (NewGGUFWriter gguf_write.go:309-442), on the host; no GPU needed.

Pinned by the reference's own cases (gguf_test.go, gguf_write_test.go): the
round-trip values, the rejected inputs, the DataSize table and the alignment
rules.  The round-trip file of TestParseGGUFRoundTrip is assembled here byte
by byte from the format description (gguf.go:3-12, cursor.value 671-767),
independently of the package's writer, so a writer and reader that agree on
a wrong layout would still fail it.
"""
import struct

import numpy as np
import pytest

from conftest import tiny_llama
from oracle import oracle as ref

gguf = pytest.importorskip("gopherllm_amd.gguf")
from gopherllm_amd.gguf import GGUFFile, GGUFWriter, MetaValue, PlannedTensor  # noqa: E402

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14


def s_(b):
    b = b.encode() if isinstance(b, str) else b
    return struct.pack("<Q", len(b)) + b


def build_gguf(version, kvs, tensors, alignment=32):
    """Spec-level builder: magic, version, counts, (key, tag, payload)...,
    (name, ndims, dims, dtype, offset)..., padding, data."""
    out = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, tag, payload in kvs:
        out += s_(key) + struct.pack("<I", tag) + payload
    off, offs = 0, []
    for _, dims, dt, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, dims, dt, data), o in zip(tensors, offs):
        out += s_(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", dt, o)
    out += bytes((-len(out)) % alignment)
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offs):
        out += bytes(base + o - len(out)) + data
    return out


def f32b(vals):
    return np.asarray(vals, np.float32).tobytes()


def test_parse_round_trip_reference_values():
    """TestParseGGUFRoundTrip (gguf_test.go:8-80)."""
    kvs = [("general.architecture", 8, s_("llama")),
           ("v.u8", 0, struct.pack("<B", 7)), ("v.i8", 1, struct.pack("<b", -3)),
           ("v.u16", 2, struct.pack("<H", 300)), ("v.i16", 3, struct.pack("<h", -300)),
           ("v.u32", 4, struct.pack("<I", 70000)), ("v.i32", 5, struct.pack("<i", -5)),
           ("v.f32", 6, struct.pack("<f", 3.5)), ("v.bool", 7, b"\x01"),
           ("v.u64", 10, struct.pack("<Q", 1 << 40)), ("v.i64", 11, struct.pack("<q", -7)),
           ("v.f64", 12, struct.pack("<d", 2.5)),
           ("toks", 9, struct.pack("<IQ", 8, 3) + s_("a") + s_("b") + s_("c")),
           ("scores", 9, struct.pack("<IQ", 6, 2) + struct.pack("<2f", 1, 2)),
           ("general.alignment", 4, struct.pack("<I", 32))]
    tensors = [("t0", [4, 2], F32, f32b([1, 2, 3, 4, 5, 6, 7, 8])),
               ("t1", [8], F32, f32b([8, 7, 6, 5, 4, 3, 2, 1]))]
    data = build_gguf(3, kvs, tensors)
    g = GGUFFile(data=data)
    assert g.version == 3
    assert g.get_str("general.architecture") == "llama"
    for k in ("v.u8", "v.i8", "v.u16", "v.u32", "v.u64"):  # AsU32 widens every integer kind
        g.get_u32(k)
    assert g.get_u32("v.u32") == 70000
    assert g.get_u32("v.i8") == (-3) & 0xffffffff and g.get_u32("v.i16") == (-300) & 0xffffffff
    assert g.get_u32("v.u64") == 0  # 1 << 40 cast to 32 bits
    assert g.get_u64("v.u64") == 1 << 40
    assert g.get_f32("v.f32") == 3.5
    assert abs(g.get_f32("v.f64") - 2.5) <= 1e-6
    assert g.get_bool("v.bool") is True
    assert g.kind("toks") == ("array", "str", 3) and g.get_str("toks", 2) == "c"
    assert g.kind("scores") == ("array", "f32", 2) and g.get_f32("scores", 1) == 2.0
    ts = g.tensors()
    assert len(ts) == 2
    assert ts[0].name == "t0" and ts[0].dims == (4, 2) and ts[0].dtype == F32 and ts[0].nbytes == 32
    assert g.data_offset % 32 == 0
    assert struct.unpack_from("<f", data, g.data_offset)[0] == 1.0
    assert np.frombuffer(g.tensor_bytes("t1"), np.float32).tolist() == [8, 7, 6, 5, 4, 3, 2, 1]
    # kinds that do not convert are refused, absent keys too
    for bad in (lambda: g.get_u32("v.f32"), lambda: g.get_f32("v.u32"),
                lambda: g.get_str("v.bool"), lambda: g.get_u32("nope"), lambda: g.get_u32("toks", 9)):
        with pytest.raises(gguf.GllmError):
            bad()


def test_parse_rejects_bad_input():
    """TestParseGGUFRejectsBadInput (gguf_test.go:82-101)."""
    for data in (bytes([1, 2]), b"XXXXwhatever"):
        with pytest.raises(gguf.GllmError):
            GGUFFile(data=data)
    valid = build_gguf(3, [("k", 4, struct.pack("<I", 1))], [])
    with pytest.raises(gguf.GllmError, match="EOF"):
        GGUFFile(data=valid[:24])  # the key is cut off
    bad = bytearray(valid)
    assert bad[24 + 8 + 1] == 4  # the value-type tag of key "k"
    bad[24 + 8 + 1] = 99
    with pytest.raises(gguf.GllmError, match="unknown GGUF value type 99"):
        GGUFFile(data=bytes(bad))
    # every proper prefix of a valid file with tensors fails cleanly
    full = build_gguf(3, [("a", 8, s_("xyz")), ("arr", 9, struct.pack("<IQ", 4, 2) + struct.pack("<2I", 5, 6))],
                      [("t", [8], F32, f32b(range(8)))])
    for cut in range(0, 100):
        try:
            GGUFFile(data=full[:cut])
        except gguf.GllmError:
            continue
        raise AssertionError(f"prefix of {cut} bytes parsed")
    # an array count larger than the file is an EOF, not an allocation
    huge = build_gguf(3, [("arr", 9, struct.pack("<IQ", 8, 1 << 60))], [])
    with pytest.raises(gguf.GllmError, match="EOF"):
        GGUFFile(data=huge)
    # an empty array of an unknown element kind carries no element to decode
    ok = GGUFFile(data=build_gguf(3, [("e", 9, struct.pack("<IQ", 77, 0))], []))
    assert ok.kind("e")[2] == 0


def test_data_size_table():
    """TestGGMLTypeDataSize (gguf_test.go:103-135)."""
    cases = [(F32, 10, 40), (F16, 10, 20), (Q8_0, 32, 34), (20, 32, 18), (22, 256, 82),
             (21, 256, 110), (23, 256, 136), (Q4_K, 256, 144), (Q6_K, 256, 210), (15, 256, 292),
             (28, 10, 80), (34, 256, 54), (35, 256, 66), (39, 32, 17), (41, 128, 18), (42, 64, 18)]
    for t, n, want in cases:
        assert gguf.data_size(t, n) == want, (t, n)
    assert gguf.data_size(255, 10) == 0


def test_unknown_type_sized_from_offsets():
    """ggmlTypeFromUint32 folds unknown ids to 255 (gguf.go:66-77); their byte
    size comes from the offset gap (inferTensorSizes, model.go:2272-2310)."""
    data = build_gguf(3, [], [("u", [10], 77, bytes(range(40))), ("f", [2], F32, f32b([1, 2]))])
    g = GGUFFile(data=data)
    u, f = g.tensors()
    assert u.dtype == 255 and u.nbytes == 64  # 40 bytes padded to the next 32-byte offset
    assert f.nbytes == 8


def test_writer_round_trip_reference_values():
    """TestGGUFWriterRoundTrip (gguf_write_test.go:15-164): every kind, both
    array representations, an F32 and a Q8_0 tensor; the Q8_0 bytes decode
    to i - 16 through the oracle's DequantRowQ8_0."""
    meta = {
        "a.u8": MetaValue("u8", 200), "a.i8": MetaValue("i8", -100), "a.u16": MetaValue("u16", 60000),
        "a.i16": MetaValue("i16", -30000), "a.u32": MetaValue("u32", 4000000000),
        "a.i32": MetaValue("i32", -2000000000), "a.f32": MetaValue("f32", 3.5),
        "a.bool_t": MetaValue("bool", True), "a.bool_f": MetaValue("bool", False),
        "a.str": MetaValue("str", "hello gguf"), "a.u64": MetaValue("u64", 18000000000000000000),
        "a.i64": MetaValue("i64", -9000000000000000000), "a.f64": MetaValue("f64", 2.718281828),
        "arr.str": MetaValue("array", ["alpha", "beta", "gamma"]),
        "arr.f32": MetaValue("array", np.array([1, 2.5, -3.25], np.float32)),
        "arr.bool": MetaValue("array", [True, False, True]),
        "arr.empty": MetaValue("array", []),
        "arr.u32": MetaValue("array", [MetaValue("u32", 10), MetaValue("u32", 20), MetaValue("u32", 30)]),
        "arr.nested": MetaValue("array", [MetaValue("array", [MetaValue("i16", -1)]),
                                          MetaValue("array", [MetaValue("i16", 2), MetaValue("i16", 3)])]),
    }
    f32 = f32b(np.arange(8) - 3.5)
    q80 = bytearray(34)
    q80[0:2] = b"\x00\x3c"  # f16 1.0
    q80[2:] = bytes((i - 16) & 0xff for i in range(32))
    planned = [PlannedTensor("tensor.f32", (8,), F32), PlannedTensor("tensor.q8_0", (32,), Q8_0)]
    import io
    buf = io.BytesIO()
    w = GGUFWriter(buf, meta, planned, 32)
    w.write_tensor(np.frombuffer(f32, np.uint8))
    w.write_tensor(np.frombuffer(bytes(q80), np.uint8))
    w.close()
    g = GGUFFile(data=buf.getvalue())
    assert g.get_u32("a.u8") == 200
    assert g.get_u32("a.i16") == (-30000) & 0xffffffff  # AsU32 widens signed via a 32-bit cast
    assert g.get_u32("a.u32") == 4000000000
    assert g.get_f32("a.f32") == 3.5
    assert g.get_bool("a.bool_t") is True and g.get_bool("a.bool_f") is False
    assert g.get_str("a.str") == "hello gguf"
    assert g.get_u64("a.u64") == 18000000000000000000
    assert g.get_u64("a.i64") == (-9000000000000000000) & (2**64 - 1)
    assert g.get_f64("a.f64") == 2.718281828
    assert [g.get_str("arr.str", i) for i in range(3)] == ["alpha", "beta", "gamma"]
    assert g.get_f32("arr.f32", 1) == 2.5 and g.get_f32("arr.f32", 2) == -3.25
    assert [g.get_bool("arr.bool", i) for i in range(3)] == [True, False, True]
    assert g.kind("arr.empty")[2] == 0
    assert [g.get_u32("arr.u32", i) for i in range(3)] == [10, 20, 30]
    assert g.kind("arr.nested") == ("array", "array", 2)
    assert g.get_u32("general.alignment") == 32
    tf, tq = g.tensors()
    assert (tf.name, tf.dtype, tf.dims) == ("tensor.f32", F32, (8,))
    assert (tq.name, tq.dtype, tq.dims) == ("tensor.q8_0", Q8_0, (32,))
    assert g.tensor_bytes("tensor.f32") == f32 and g.tensor_bytes("tensor.q8_0") == bytes(q80)
    deq = ref.dequant_row(ref.Q8_0, np.frombuffer(bytes(q80), np.uint8), 32)
    assert deq.tolist() == [float(i - 16) for i in range(32)]


def test_writer_alignment_and_short_tensor():
    """TestGGUFWriterAlignment / RejectsShortTensor (gguf_write_test.go:172-212)."""
    import io
    buf = io.BytesIO()
    w = GGUFWriter(buf, {"k": MetaValue("str", "v")}, [PlannedTensor("t", (32,), Q8_0)], 64)
    w.write_tensor(np.zeros(34, np.uint8))
    w.close()
    g = GGUFFile(data=buf.getvalue())
    assert g.data_offset % 64 == 0
    assert len(buf.getvalue()) == g.data_offset + 34  # no pad after the last tensor
    w = GGUFWriter(io.BytesIO(), {}, [PlannedTensor("t", (32,), Q8_0)], 32)
    with pytest.raises(ValueError):
        w.write_tensor(np.zeros(10, np.uint8))
    with pytest.raises(ValueError):
        w.close()


def test_llama_file_layout(tmp_path):
    """write_llama_gguf: llama.cpp names, dims in GGUF order (cols first), and
    every tensor's bytes as given, read back through the mapping."""
    m = tiny_llama(seed=9, n_layers=2, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=300)
    path = gguf.write_llama_gguf(tmp_path / "tiny.gguf", m)
    with GGUFFile(path) as g:
        assert g.get_str("general.architecture") == "llama"
        assert g.get_u32("llama.block_count") == 2 and g.get_u32("llama.embedding_length") == 256
        assert g.get_u32("llama.attention.head_count_kv") == 1
        assert g.get_f32("llama.rope.freq_base") == 500000.0
        names = [t.name for t in g.tensors()]
        assert names[:3] == ["token_embd.weight", "output_norm.weight", "output.weight"]
        assert "blk.1.ffn_down.weight" in names
        t = g.tensors()[g.find("blk.1.ffn_down.weight")]
        assert t.dims == (512, 256) and t.dtype == Q4_K and t.offset % 32 == 0
        assert g.tensor_bytes("blk.1.ffn_down.weight") == np.asarray(m["w2"][1]).tobytes()
        assert g.tensor_bytes("output.weight") == np.asarray(m["output"]).tobytes()
        assert np.frombuffer(g.tensor_bytes("blk.0.attn_norm.weight"), np.float32).tolist() == [1.0] * 256
    with pytest.raises(gguf.GllmError):
        GGUFFile(tmp_path / "missing.gguf")


REFUSED = [
    ("llama.rope.dimension_count", ("u32", 32)),
    ("llama.attention.value_length", ("u32", 32)),
    ("llama.attention.temperature_scale", ("f32", 0.1)),
    ("llama.attention.sliding_window", ("u32", 16)),
    ("llama.attn_logit_softcapping", ("f32", 30.0)),
    ("llama.final_logit_softcapping", ("f32", 30.0)),
    ("llama.embedding_scale", ("f32", 2.0)),
    ("llama.residual_scale", ("f32", 0.5)),
    ("llama.logit_scale", ("f32", 0.5)),
    ("yarn", None),
    ("rope_factors_long.weight", None),
]


@pytest.mark.parametrize("key,value", REFUSED, ids=[k for k, _ in REFUSED])
def test_model_from_gguf_refuses_graph_changing_keys(tmp_path, key, value):
    """Keys of ConfigFromGGUF / LoadModel (model.go:400-452, 1728-1756,
    1866-1869) that change the llama graph away from the plain one this
    decoder runs make gllm_hip_model_from_gguf fail with GLLM_EUNSUP, naming
    the key, before any device work (so this runs without a GPU)."""
    from conftest import tiny_llama
    from gopherllm_amd import _lib, gguf
    m = tiny_llama(seed=2, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=300)
    extra, tensors = {}, ()
    if key == "yarn":
        extra = {"llama.rope.scaling.type": gguf.MetaValue("str", "yarn"),
                 "llama.rope.scaling.factor": gguf.MetaValue("f32", 4.0),
                 "llama.rope.scaling.original_context_length": gguf.MetaValue("u32", 1024)}
    elif key.endswith(".weight"):
        tensors = ((key, (32,), 0, np.ones(32, np.float32)),)
    else:
        extra = {key: gguf.MetaValue(*value)}
    path = gguf.write_llama_gguf(tmp_path / "x.gguf", m, extra_meta=extra, extra_tensors=tensors)
    f = gguf.GGUFFile(str(path))
    L = _lib.load()
    h = L.gllm_hip_model_from_gguf(f.handle, 64)
    assert not h
    msg = _lib.last_error()
    assert "not supported" in msg and (key.split(".")[-1] in msg or key in msg), msg
    f.close()


@pytest.mark.parametrize("rope_dim", [("u32", 64), ("u32", 0), ("u32", 128), ("i32", -1)])
def test_model_from_gguf_accepts_default_valued_keys(tmp_path, rope_dim):
    """The same keys at their defaults (rope over the whole head, value
    length = head_dim, unit scales, no window) pass the check: the call then
    fails only where this host has no device, not on the key check.  A rope
    dimension count of 0, below 0 or above head_dim means the whole head
    (buildRopeInvFreq, model.go:1729-1732), so it passes too."""
    from conftest import tiny_llama
    from gopherllm_amd import _lib, gguf
    m = tiny_llama(seed=2, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=300)
    extra = {"llama.rope.dimension_count": gguf.MetaValue(*rope_dim),
             "llama.attention.value_length": gguf.MetaValue("u32", 64),
             "llama.residual_scale": gguf.MetaValue("f32", 1.0),
             "llama.logit_scale": gguf.MetaValue("f32", 1.0),
             "llama.attention.sliding_window": gguf.MetaValue("u32", 0)}
    path = gguf.write_llama_gguf(tmp_path / "ok.gguf", m, extra_meta=extra)
    f = gguf.GGUFFile(str(path))
    L = _lib.load()
    h = L.gllm_hip_model_from_gguf(f.handle, 64)
    if h:
        L.gllm_hip_model_release(h)
    else:
        assert "not supported" not in _lib.last_error(), _lib.last_error()
    f.close()
