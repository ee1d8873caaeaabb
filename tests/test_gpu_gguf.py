"""GGUF load path on the device: weights uploaded from the file mapping
(loadWeight model.go:2357-2476) and the resident llama decoder built from a
file (LoadModel model.go:1872-1930) give the same bits and tokens as the
oracle on the same tensors."""
import numpy as np
import pytest

from conftest import normal, q4km_types, quant_matrix, tiny_llama
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def varied_norms(m, seed):
    rng = np.random.default_rng(seed)
    m["out_norm"] = (1 + 0.2 * rng.standard_normal(m["config"]["dim"])).astype(np.float32)
    m["attn_norm"] = [(1 + 0.2 * rng.standard_normal(m["config"]["dim"])).astype(np.float32)
                      for _ in m["attn_norm"]]
    m["ffn_norm"] = [(1 + 0.2 * rng.standard_normal(m["config"]["dim"])).astype(np.float32)
                     for _ in m["ffn_norm"]]
    return m


def test_decoder_from_gguf_matches_oracle(hip, tmp_path):
    from gopherllm_amd import gguf
    from gopherllm_amd.decoder import LlamaDecoder
    m = varied_norms(tiny_llama(seed=31, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2,
                                head_dim=64, vocab=2500), 32)
    path = gguf.write_llama_gguf(tmp_path / "m.gguf", m)
    prompt = np.random.default_rng(33).integers(0, 2500, 40)
    print("from_gguf generate", flush=True)
    dec = LlamaDecoder.from_gguf(str(path), 96)
    got = dec.generate(prompt, 16)
    cpu = ref.Llama(m, 96)
    want = cpu.generate(prompt, 16)
    assert np.array_equal(got, want), (got, want)
    kv = dec.kv_cache()
    used = len(prompt) + 15
    for l in range(2):
        k, v = kv.read(l, 0, used)
        assert np.array_equal(k, cpu.kcache(l, 96)[:used])
        assert np.array_equal(v, cpu.vcache(l, 96)[:used])
    dec.release()


def test_decoder_from_gguf_tied_output(hip, tmp_path):
    """No output.weight: the head is token_embd (model.go:1888-1899)."""
    from gopherllm_amd import gguf
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=34, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=1200)
    m["output"] = None
    path = gguf.write_llama_gguf(tmp_path / "tied.gguf", m)
    tied = dict(m)
    tied["output"] = m["tok_embd"]
    tied["config"] = dict(m["config"], out_type=m["config"]["emb_type"])
    prompt = np.random.default_rng(35).integers(0, 1200, 20)
    dec = LlamaDecoder.from_gguf(str(path), 64)
    assert np.array_equal(dec.generate(prompt, 10), ref.Llama(tied, 64).generate(prompt, 10))


@pytest.mark.parametrize("qtype", [ref.Q4_K, ref.Q6_K, ref.Q8_0])
def test_load_weight_from_mapping(hip, tmp_path, qtype):
    from gopherllm_amd.gguf import GGUFFile, GGUFWriter, PlannedTensor
    rows, cols = 300, 1024
    data, _ = quant_matrix(qtype, rows, cols, 36 + qtype)
    path = tmp_path / "w.gguf"
    with open(path, "wb") as f:
        w = GGUFWriter(f, {}, [PlannedTensor("w", (cols, rows), qtype)], 32)
        w.write_tensor(data)
        w.close()
    x = normal(37, cols)
    with GGUFFile(path) as g:
        wt = g.load_weight("w")
        assert (wt.rows, wt.cols, wt.type) == (rows, cols, qtype)
        got = wt.matvec_into(x)
    want = hip.Weight.from_host(data, qtype, rows, cols).matvec_into(x)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(got), bits(ref.matvec(qtype, data, x, rows, cols)))


def test_truncated_weight_is_zero_padded(hip, tmp_path):
    """loadWeight pads a quantised tensor the file cuts short with zeros."""
    from gopherllm_amd.gguf import GGUFFile, GGUFWriter, PlannedTensor
    rows, cols = 64, 512
    data, _ = quant_matrix(ref.Q4_K, rows, cols, 38)
    path = tmp_path / "short.gguf"
    with open(path, "wb") as f:
        w = GGUFWriter(f, {}, [PlannedTensor("w", (cols, rows), ref.Q4_K)], 32)
        w.write_tensor(data)
        w.close()
    raw = path.read_bytes()
    keep = len(raw) - 10 * 288 - 100  # drop the last 10.x rows
    path.write_bytes(raw[:keep])
    with GGUFFile(path) as g:
        got = g.load_weight("w").matvec_into(normal(39, cols))
    nbytes = len(data)
    off = len(raw) - nbytes  # the single tensor ends the file
    zp = np.zeros(nbytes, np.uint8)
    zp[:keep - off] = np.frombuffer(raw[off:keep], np.uint8)
    want = ref.matvec(ref.Q4_K, zp, normal(39, cols), rows, cols)
    assert np.array_equal(bits(got), bits(want))
    assert np.all(got[-10:] == 0.0)


def test_decoder_from_mixed_gguf_matches_oracle(hip, tmp_path):
    """A Q4_K_M-style file (Q6_K attn_v / ffn_down on some layers): each
    tensor is uploaded with its own type tag and the decoder's mixed
    projection groups give the oracle's tokens."""
    from gopherllm_amd import gguf
    from gopherllm_amd.decoder import LlamaDecoder
    m = varied_norms(tiny_llama(seed=35, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2,
                                head_dim=64, vocab=900, type_of=q4km_types), 36)
    path = gguf.write_llama_gguf(tmp_path / "mixed.gguf", m)
    with gguf.GGUFFile(str(path)) as f:
        types = {t.name: t.dtype for t in f.tensors()}
    assert types["blk.0.attn_v.weight"] == ref.Q6_K and types["blk.0.ffn_down.weight"] == ref.Q6_K
    assert types["blk.1.attn_v.weight"] == ref.Q4_K and types["blk.0.attn_q.weight"] == ref.Q4_K
    prompt = np.random.default_rng(37).integers(0, 900, 24)
    print("from_gguf mixed generate", flush=True)
    dec = LlamaDecoder.from_gguf(str(path), 64)
    got = dec.generate(prompt, 10)
    want = ref.Llama(m, 64).generate(prompt, 10)
    assert np.array_equal(got, want), (got, want)
    dec.release()


def test_decoder_from_gguf_attention_scale(hip, tmp_path):
    """llama.attention.scale replaces 1/sqrt(head_dim) (config.AttentionScale,
    model.go:2685-2688): tokens and KV rows equal the oracle run with the
    same scale, and differ from the default-scale run."""
    from gopherllm_amd import gguf
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=36, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2,
                   head_dim=64, vocab=1500)
    m["config"] = dict(m["config"], attn_scale=0.5)
    path = gguf.write_llama_gguf(tmp_path / "scale.gguf", m)
    prompt = np.random.default_rng(37).integers(0, 1500, 30)
    print("from_gguf attention.scale generate", flush=True)
    dec = LlamaDecoder.from_gguf(str(path), 64)
    got = dec.generate(prompt, 12)
    cpu = ref.Llama(m, 64)
    want = cpu.generate(prompt, 12)
    assert np.array_equal(got, want), (got, want)
    k, _ = dec.kv_cache().read(1, 0, 41)
    assert np.array_equal(k, cpu.kcache(1, 64)[:41])
    default = dict(m, config=dict(m["config"], attn_scale=0.0))
    cpu0 = ref.Llama(default, 64)
    cpu0.generate(prompt, 12)
    assert not np.array_equal(cpu0.kcache(1, 64)[:41], k)
    dec.release()
