"""Resident decoder parity: hidden states, KV cache rows and greedy tokens of
the device llama graph are identical to the oracle's restatement of
ForwardBodyInto / ForwardBatchInto on the same weights."""
import numpy as np
import pytest

from conftest import q4km_types, tiny_llama
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_decode_steps_bit_exact(hip):
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=3, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2, head_dim=64,
                   vocab=2000)
    max_len = 64
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    tok = 7
    for pos in range(12):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


def test_captured_decode_long_cache_bit_exact(hip):
    """A cache longer than the one-token values kernel's LDS image (4000 >
    3272 positions, head_dim 128): the captured decode step runs the
    long-span values kernel with the span read on the device, from one
    position through spans past one 128-position staging step; hidden
    states and greedy tokens identical to the oracle's."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=21, n_layers=2, dim=512, hidden=1024, n_heads=4, n_kv_heads=1,
                   head_dim=128, vocab=1000)
    max_len = 4000
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    tok = 11
    for pos in range(136):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


def test_captured_decode_past_eager_rows_bit_exact(hip):
    """Captured decode steps at spans past 2048 positions in a 4000-position
    cache: the scores chunks past the first 2048 rows read the position
    before loading, those inside the span score their rows and those past it
    leave at once; hidden states and greedy tokens identical to the oracle's
    after a 2100-token prefill."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=22, n_layers=2, dim=512, hidden=1024, n_heads=4, n_kv_heads=1,
                   head_dim=128, vocab=1000)
    max_len = 4000
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    prompt = np.random.default_rng(23).integers(0, 1000, 2100)
    print("long-cache prefill 2100 tokens", flush=True)
    gt = gpu.prefill(prompt)
    ct, _ = cpu.prefill(prompt)
    assert gt == ct
    tok = ct
    for pos in range(2100, 2104):
        print(f"long-cache decode pos {pos}", flush=True)
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


def test_prefill_then_decode_tokens_identical(hip):
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=4, n_layers=3, dim=512, hidden=1536, n_heads=8, n_kv_heads=2, head_dim=64,
                   vocab=3000)
    prompt = np.random.default_rng(5).integers(0, 3000, 70)
    max_len = 128
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    want = cpu.generate(prompt, 24)
    got = gpu.generate(prompt, 24)
    assert np.array_equal(got, want), (got, want)
    # the KV cache rows written by prefill + decode are bit-identical
    kv = gpu.kv_cache()
    used = len(prompt) + 23
    for l in range(3):
        k, v = kv.read(l, 0, used)
        assert np.array_equal(k, cpu.kcache(l, max_len)[:used])
        assert np.array_equal(v, cpu.vcache(l, max_len)[:used])


def test_prefill_logits_match_oracle(hip):
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=6, n_layers=2, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=1500)
    prompt = np.random.default_rng(7).integers(0, 1500, 100)
    gpu = LlamaDecoder.from_host_model(m, 160)
    cpu = ref.Llama(m, 160)
    gt, gl = gpu.prefill(prompt, want_logits=True)
    ct, cl = cpu.prefill(prompt)
    assert gt == ct
    assert np.array_equal(bits(gl), bits(cl))


def test_generate_with_repeat_penalty(hip):
    """forwardGreedyToken with recent / repeatPenalty (runtime.go:1607): the
    window holds the last tokens seen (prompt, then each emitted token,
    runtime.go:1035, 1089-1093) and every greedy choice applies
    applyRepeatPenalty (sampling.go:136-153).  Plain greedy on this model
    repeats one token; the penalties break that, and a window of 8 lets the
    token return once it has slid out; a window of 90 holds more ids than
    one wave's lanes.  Decode steps after the first replay the captured step
    graph, so the window reaches it through device memory."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=4, n_layers=3, dim=512, hidden=1536, n_heads=8, n_kv_heads=2, head_dim=64,
                   vocab=3000)
    prompt = np.random.default_rng(5).integers(0, 3000, 70)
    gpu = LlamaDecoder.from_host_model(m, 128)
    plain = ref.Llama(m, 128).generate(prompt, 24)
    for pen, win in ((1.8, 64), (4.0, 8), (0.7, 16), (1.0, 64), (1.3, 90)):
        print(f"repeat penalty {pen} window {win}", flush=True)
        cpu = ref.Llama(m, 128)
        cpu.set_repeat_penalty(pen, win)
        want = cpu.generate(prompt, 24)
        gpu.set_repeat_penalty(pen, win)
        got = gpu.generate(prompt, 24)
        assert np.array_equal(got, want), (pen, win, got, want)
        if pen > 1.0:
            assert not np.array_equal(got, plain)
    with pytest.raises(hip.GllmError):
        gpu.set_repeat_penalty(0.0, 64)
    with pytest.raises(hip.GllmError):
        gpu.set_repeat_penalty(1.5, -1)


def test_back_to_back_requests_do_not_share_the_penalty_window(hip):
    """Each request's window is the tail of its own prompt
    (recentTokenWindowInto, runtime.go:1035): a second request on the same
    model, prefilled from position 0 without another set_repeat_penalty,
    chooses what a fresh oracle chooses for that prompt alone; a request
    after set_repeat_penalty(1) is plain greedy."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=4, n_layers=3, dim=512, hidden=1536, n_heads=8, n_kv_heads=2, head_dim=64,
                   vocab=3000)
    rng = np.random.default_rng(15)
    pa, pb = rng.integers(0, 3000, 50), rng.integers(0, 3000, 40)
    gpu = LlamaDecoder.from_host_model(m, 128)

    def fresh(prompt, pen, win):
        cpu = ref.Llama(m, 128)
        if pen != 1.0:
            cpu.set_repeat_penalty(pen, win)
        return cpu.generate(prompt, 20)

    gpu.set_repeat_penalty(2.5, 16)
    print("request A, penalty 2.5 window 16", flush=True)
    assert np.array_equal(gpu.generate(pa, 20), fresh(pa, 2.5, 16))
    print("request B, same setting, no reset", flush=True)
    assert np.array_equal(gpu.generate(pb, 20), fresh(pb, 2.5, 16))
    gpu.set_repeat_penalty(1.0, 64)
    print("request A again, penalty 1", flush=True)
    assert np.array_equal(gpu.generate(pa, 20), fresh(pa, 1.0, 64))


def test_decode_8b_layer_shapes_bit_exact(hip):
    """Two layers at the 8B shapes (dim 4096, hidden 14336, 32 / 8 heads of
    128), the row kernels the full model runs (fused-quantiser Q4_K at 4096
    columns, 14336-column down projection), non-trivial norm weights: hidden
    states and greedy tokens identical to the oracle's ForwardBodyInto
    through prefill and the captured, replayed decode step."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=12, n_layers=2, dim=4096, hidden=14336, n_heads=32, n_kv_heads=8,
                   head_dim=128, vocab=1200)
    rng = np.random.default_rng(13)
    m["out_norm"] = (1 + 0.2 * rng.standard_normal(4096)).astype(np.float32)
    m["attn_norm"] = [(1 + 0.2 * rng.standard_normal(4096)).astype(np.float32) for _ in range(2)]
    m["ffn_norm"] = [(1 + 0.2 * rng.standard_normal(4096)).astype(np.float32) for _ in range(2)]
    max_len = 64
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len, fast=True)
    prompt = rng.integers(0, 1200, 9)
    gt = gpu.prefill(prompt)
    ct, _ = cpu.prefill(prompt)
    assert gt == ct
    tok = gt
    for i in range(12):
        pos = len(prompt) + i
        print(f"8b-shape decode pos {pos}", flush=True)
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


def test_mixed_q4k_q6k_layers_match_oracle(hip):
    """A Q4_K_M-style model (Q6_K attn_v / ffn_down in some layers): every
    projection is its own int8 row dot, as in the reference's mixed groups
    (tryMatvecAttentionInto, model.go:3156-3190; matvecBatchQ8Fused for
    prefill), so prefill logits, decode hidden states and greedy tokens are
    bit-identical to the oracle's."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=12, n_layers=3, dim=512, hidden=1024, n_heads=8, n_kv_heads=2,
                   head_dim=64, vocab=1200, type_of=q4km_types)
    prompt = np.random.default_rng(13).integers(0, 1200, 40)
    max_len = 96
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    print("mixed-type model: prefill", flush=True)
    gt, gl = gpu.prefill(prompt, want_logits=True)
    ct, cl = cpu.prefill(prompt)
    assert np.array_equal(bits(gl), bits(cl))
    assert gt == ct
    tok = ct
    for pos in range(len(prompt), len(prompt) + 8):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


def test_q4k_pair_with_a_q8_0_projection_matches_oracle(hip):
    """Q/K/V = Q4_K, Q8_0, Q4_K: the Q4_K pair (0, 2) is the fused group and
    runs the int8 row dots, the Q8_0 K its own MatvecInto
    (tryMatvecAttentionInto, model.go:3157-3184)."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=14, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1,
                   head_dim=64, vocab=300,
                   type_of=lambda l, k: ref.Q8_0 if k == "wk" else ref.Q4_K)
    gpu = LlamaDecoder.from_host_model(m, 32)
    cpu = ref.Llama(m, 32)
    tok = 1
    for pos in range(6):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


@pytest.mark.parametrize("n_heads,n_kv", [(8, 2), (4, 4), (8, 4), (8, 1)])
def test_decode_attention_head_dim_128_matches_oracle(hip, n_heads, n_kv):
    """head_dim 128 generation steps (captured decode step: RoPE and the
    K / V store folded into the scores stage, scores and values in one
    launch for up to 4 query heads per KV head, the value chains over V rows
    staged through LDS): hidden states, tokens and the cache rows equal the
    oracle's, for spans that cross the 64-position tiles, with 1, 2, 4 and 8
    query heads per KV head."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=31, n_layers=2, dim=512, hidden=1024, n_heads=n_heads, n_kv_heads=n_kv,
                   head_dim=128, vocab=700)
    max_len = 200
    prompt = np.random.default_rng(32).integers(0, 700, 60)
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    gt = gpu.prefill(prompt)
    ct, _ = cpu.prefill(prompt)
    assert gt == ct
    tok = ct
    for pos in range(len(prompt), len(prompt) + 75):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want
    kv = gpu.kv_cache()
    used = len(prompt) + 75
    for l in range(2):
        k, v = kv.read(l, 0, used)
        assert np.array_equal(k, cpu.kcache(l, max_len)[:used])
        assert np.array_equal(v, cpu.vcache(l, max_len)[:used])


def test_swiglu_epilogue_decode_matches_oracle(hip):
    """dim 1024, hidden 8192: the gate/up launch takes the RMSNorm prologue
    and the SwiGLU + Q8K epilogue (the last workgroup of each 256-row block
    quantises it for the down projection, block counters reset for the next
    step), over repeated graph replays; hidden states and tokens equal the
    oracle's."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=41, n_layers=2, dim=1024, hidden=8192, n_heads=8, n_kv_heads=2,
                   head_dim=128, vocab=500)
    max_len = 48
    prompt = np.random.default_rng(42).integers(0, 500, 9)
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    gt = gpu.prefill(prompt)
    ct, _ = cpu.prefill(prompt)
    assert gt == ct
    tok = ct
    for pos in range(len(prompt), len(prompt) + 12):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want


def test_prompt_longer_than_one_prefill_chunk(hip):
    """A 700-token prompt runs as two prefill chunks (512 + 188 tokens; the
    second attends over the first chunk's KV rows), then 8 greedy steps:
    tokens, the prompt's last logits and every KV row equal the oracle's."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=13, n_layers=2, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=1200)
    prompt = np.random.default_rng(14).integers(0, 1200, 700)
    max_len = 768
    print("700-token prompt, two chunks", flush=True)
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    gt, gl = gpu.prefill(prompt, want_logits=True)
    ct, cl = cpu.prefill(prompt)
    assert gt == ct
    assert np.array_equal(bits(gl), bits(cl))
    g2 = LlamaDecoder.from_host_model(m, max_len)
    c2 = ref.Llama(m, max_len)
    want = c2.generate(prompt, 8)
    got = g2.generate(prompt, 8)
    assert np.array_equal(got, want), (got, want)
    kv = g2.kv_cache()
    used = len(prompt) + 7
    for l in range(2):
        k, v = kv.read(l, 0, used)
        assert np.array_equal(k, c2.kcache(l, max_len)[:used]), l
        assert np.array_equal(v, c2.vcache(l, max_len)[:used]), l


def test_prefill_crossing_position_6144(hip):
    """A 300-token prefill at positions 6000..6299 over a cache whose rows
    0..5999 hold the same random f16 K/V on both sides: its later tokens span
    more than 6144 positions, where prefill attention takes the generic
    scores / softmax / values kernels (in the model's scores buffer).  The
    logits, the token, the new KV rows and 4 decode steps after it equal the
    oracle's."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=15, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=1200)
    max_len, start, n = 6400, 6000, 300
    kvd = 64
    rng = np.random.default_rng(16)
    k = rng.standard_normal((start, kvd), dtype=np.float32)
    v = rng.standard_normal((start, kvd), dtype=np.float32)
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    print(f"fill KV rows 0..{start - 1}", flush=True)
    kv = gpu.kv_cache()
    for p in range(start):
        kv.store_kv(0, p, k[p], v[p])
    cpu.set_kv(0, 0, ref.f32_to_f16(k), ref.f32_to_f16(v))
    prompt = rng.integers(0, 1200, n)
    print(f"prefill {n} tokens at {start}", flush=True)
    gt, gl = gpu.prefill(prompt, start_pos=start, want_logits=True)
    ct, cl = cpu.prefill(prompt, start_pos=start)
    assert gt == ct
    assert np.array_equal(bits(gl), bits(cl))
    gk, gv = kv.read(0, 0, start + n)
    assert np.array_equal(gk, cpu.kcache(0, max_len)[:start + n])
    assert np.array_equal(gv, cpu.vcache(0, max_len)[:start + n])
    tok = gt
    for pos in range(start + n, start + n + 4):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert got == want, pos
        tok = want


def test_prefill_mixed_types_take_the_batched_tiles(hip):
    """Q4_K_M-style mix at widths whose rows hold a multiple of 8 blocks
    (dim 2048, hidden 4096): the prefill's Q6_K attn_v / ffn_down run the
    matrix-core tiles and a Q8_0 ffn_down the vector-unit tiles (prompt of
    90 tokens: ragged 64-token tiles), then greedy steps; logits, hidden
    states and tokens equal the oracle's."""
    from gopherllm_amd.decoder import LlamaDecoder

    def types(l, name):
        if name == "w2" and l == 1:
            return ref.Q8_0
        return q4km_types(l, name)

    m = tiny_llama(seed=51, n_layers=2, dim=2048, hidden=4096, n_heads=16, n_kv_heads=4,
                   head_dim=128, vocab=600, type_of=types)
    prompt = np.random.default_rng(52).integers(0, 600, 90)
    max_len = 104
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    print("mixed-type model, tiled prefill", flush=True)
    gt, gl = gpu.prefill(prompt, want_logits=True)
    ct, cl = cpu.prefill(prompt)
    assert np.array_equal(bits(gl), bits(cl))
    assert gt == ct
    tok = ct
    for pos in range(len(prompt), len(prompt) + 4):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert np.array_equal(bits(gpu.hidden()), bits(hid)), pos
        assert got == want, pos
        tok = want
