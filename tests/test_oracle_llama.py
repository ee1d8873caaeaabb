"""Pins the oracle's llama decoder composition (ref_llama_prefill / _decode,
oracle/gllm_oracle.c llama_body) against an independent float64 forward.

The oracle's primitives (row dots, Q8K, RMSNorm, RoPE, attention, SiLU) are
pinned one by one in test_oracle.py.  What those tests leave open is how
ForwardBodyInto (model.go:2622-2820) wires them together: which norm weight
feeds which projection, RoPE on q and on k (interleaved pairs,
applyPreparedRope model.go:3051-3093), the GQA map (query head h reads kv
head h / kvMul, model.go:2830), the causal range 0..pos, both residual adds
(addInPlace, model.go:2712 and 2813), SwiGLU (siluMulF32) and the final norm
before the output head.  `Float64Llama` below is a textbook statement of
that graph in float64 on the dequantised weights (DequantRow*Into), with no
int8 activations; the oracle quantises every activation to Q8K, so the two
agree to a stated tolerance, not bitwise:

  * KV_TOL: relative L2 error of each layer's K rows and V rows (all
    prompt and decode positions, f16 as stored).  Measured at 0.8-3.8e-2 on
    these models (Q8K activation rounding, growing with depth), so the bar
    is 6e-2.  The K / V rows pin each layer separately: layer l's rows see
    everything layers 0..l-1 computed.
  * OUT_TOL: relative L2 error of the prompt's last-position logits and of
    every decode step's output-normed hidden state.  Measured at up to
    5e-2 (peaked attention amplifies the activation rounding), so the bar
    is 1e-1.
  * every mutation in MUTATIONS (a plausible composition mistake planted in
    the float64 forward, on the CPU) moves the K / V rows or the outputs by
    more than 3x their tolerance on every config where it changes the
    function; the test asserts that too, so the tolerances are shown to be
    tight enough to see each mistake.

The models are chosen so that these mistakes are visible: wq / wk are drawn
wider than the N(0, 0.02) benchmark weights so that attention is far from
uniform (with near-uniform weights RoPE and the GQA map barely matter), and
the norm weights are random and distinct per slot.

Structural invariants of the oracle itself follow at the end: KV rows past
the current position do not reach the output (causality), zero wo / w2
leave the output-normed embedding (residual wiring), and renumbering the kv
heads together with their query groups leaves every logit unchanged to
float rounding (GQA map).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import normal
from oracle import oracle as ref

KV_TOL = 6e-2
OUT_TOL = 1e-1

# (layers, dim, hidden, q heads, kv heads, head dim, vocab, layer type)
CONFIGS = [
    dict(seed=21, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2, head_dim=64,
         vocab=700, layer_type=ref.Q4_K),
    dict(seed=22, n_layers=3, dim=256, hidden=768, n_heads=4, n_kv_heads=4, head_dim=64,
         vocab=500, layer_type=ref.Q6_K),
    dict(seed=23, n_layers=2, dim=512, hidden=768, n_heads=8, n_kv_heads=1, head_dim=64,
         vocab=600, layer_type=ref.Q8_0),
]

MUTATIONS = ("no_rope_k", "no_rope_q", "rope_half_split", "gqa_modulo", "causal_one_short",
             "drop_attn_residual", "drop_ffn_residual", "swap_norms", "no_final_norm",
             "silu_on_up", "scale_sqrt_dim")

STD = {"wq": 0.08, "wk": 0.08, "wv": 0.05, "wo": 0.05, "w1": 0.04, "w2": 0.04, "w3": 0.04}


def sensitive_llama(seed, n_layers, dim, hidden, n_heads, n_kv_heads, head_dim, vocab,
                    layer_type, out_type=ref.Q6_K):
    """A llama-shaped model dict (the oracle.Llama form) whose attention is
    peaked and whose norm weights differ per slot."""
    cfg = dict(n_layers=n_layers, dim=dim, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv_heads,
               head_dim=head_dim, vocab=vocab, rms_eps=1e-5, rope_theta=10000.0,
               emb_type=ref.Q4_K, out_type=out_type, layer_type=layer_type)
    qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
    s = seed * 1000
    rng = np.random.default_rng(s)
    m = {"config": cfg}
    m["tok_embd"] = ref.quantize_rows(ref.Q4_K, normal(s + 1, (vocab, dim), 1.0))
    m["output"] = ref.quantize_rows(out_type, normal(s + 2, (vocab, dim), 0.05))
    m["out_norm"] = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    shapes = {"wq": (qd, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, qd),
              "w1": (hidden, dim), "w2": (dim, hidden), "w3": (hidden, dim)}
    for i, (k, (r, c)) in enumerate(shapes.items()):
        m[k] = [ref.quantize_rows(layer_type, normal(s + 10 + 10 * l + i, (r, c), STD[k]))
                for l in range(n_layers)]
    m["attn_norm"] = [rng.uniform(0.5, 1.5, dim).astype(np.float32) for _ in range(n_layers)]
    m["ffn_norm"] = [rng.uniform(0.5, 1.5, dim).astype(np.float32) for _ in range(n_layers)]
    return m


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


class Float64Llama:
    """Textbook llama decode in float64 on dequantised weights (the graph of
    ForwardBodyInto, model.go:2622-2820, for the plain llama architecture).
    `mutation` plants one composition mistake (for the sensitivity check)."""

    def __init__(self, m, max_len, mutation=None):
        c = m["config"]
        self.c, self.mut = c, mutation
        self.hd = c["head_dim"]
        self.kvmul = c["n_heads"] // c["n_kv_heads"]
        dq = lambda t, d, r, k: ref.dequant(t, d, r, k).astype(np.float64)  # noqa: E731
        dim, hid = c["dim"], c["hidden"]
        qd, kvd = c["n_heads"] * self.hd, c["n_kv_heads"] * self.hd
        lt = c["layer_type"]
        self.emb = dq(c["emb_type"], m["tok_embd"], c["vocab"], dim)
        self.out = dq(c["out_type"], m["output"], c["vocab"], dim)
        self.layers = []
        for l in range(c["n_layers"]):
            self.layers.append(dict(
                wq=dq(lt, m["wq"][l], qd, dim), wk=dq(lt, m["wk"][l], kvd, dim),
                wv=dq(lt, m["wv"][l], kvd, dim), wo=dq(lt, m["wo"][l], dim, qd),
                w1=dq(lt, m["w1"][l], hid, dim), w2=dq(lt, m["w2"][l], dim, hid),
                w3=dq(lt, m["w3"][l], hid, dim),
                an=np.asarray(m["attn_norm"][l], np.float64),
                fn=np.asarray(m["ffn_norm"][l], np.float64)))
        self.on = np.asarray(m["out_norm"], np.float64)
        self.K = np.zeros((c["n_layers"], max_len, c["n_kv_heads"], self.hd))
        self.V = np.zeros_like(self.K)
        self.xn = None

    def norm(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c["rms_eps"]) * w

    def rope(self, v, n_heads, pos):
        hd = self.hd
        inv = self.c["rope_theta"] ** (-np.arange(0, hd, 2) / hd)
        ang = pos * inv
        cs, sn = np.cos(ang), np.sin(ang)
        v = v.reshape(n_heads, hd).copy()
        if self.mut == "rope_half_split":  # NeoX halves instead of interleaved pairs
            a, b = v[:, :hd // 2].copy(), v[:, hd // 2:].copy()
            v[:, :hd // 2], v[:, hd // 2:] = a * cs - b * sn, a * sn + b * cs
        else:
            a, b = v[:, 0::2].copy(), v[:, 1::2].copy()
            v[:, 0::2], v[:, 1::2] = a * cs - b * sn, a * sn + b * cs
        return v.reshape(-1)

    def step(self, token, pos):
        c, hd, mut = self.c, self.hd, self.mut
        x = self.emb[token].copy()
        for l, L in enumerate(self.layers):
            an, fn = (L["fn"], L["an"]) if mut == "swap_norms" else (L["an"], L["fn"])
            xn = self.norm(x, an)
            q, k, v = L["wq"] @ xn, L["wk"] @ xn, L["wv"] @ xn
            if mut != "no_rope_q":
                q = self.rope(q, c["n_heads"], pos)
            if mut != "no_rope_k":
                k = self.rope(k, c["n_kv_heads"], pos)
            # the cache holds f16 rows (storeKV, model.go:1466-1489)
            self.K[l, pos] = k.reshape(-1, hd).astype(np.float16).astype(np.float64)
            self.V[l, pos] = v.reshape(-1, hd).astype(np.float16).astype(np.float64)
            end = pos if mut == "causal_one_short" and pos > 0 else pos + 1
            scale = 1.0 / np.sqrt(c["dim"] if mut == "scale_sqrt_dim" else hd)
            attn = np.empty(c["n_heads"] * hd)
            for h in range(c["n_heads"]):
                g = h % c["n_kv_heads"] if mut == "gqa_modulo" else h // self.kvmul
                s = self.K[l, :end, g] @ q[h * hd:(h + 1) * hd] * scale
                w = np.exp(s - s.max())
                attn[h * hd:(h + 1) * hd] = (w / w.sum()) @ self.V[l, :end, g]
            o = L["wo"] @ attn
            x = o if mut == "drop_attn_residual" else x + o
            xn2 = self.norm(x, fn)
            gate, up = L["w1"] @ xn2, L["w3"] @ xn2
            if mut == "silu_on_up":
                gate, up = up, gate
            hidden = gate / (1.0 + np.exp(-gate)) * up
            d = L["w2"] @ hidden
            x = d if mut == "drop_ffn_residual" else x + d
        self.xn = x.copy() if mut == "no_final_norm" else self.norm(x, self.on)
        return self.xn

    def logits(self):
        return self.out @ self.xn


def run_float64(m, prompt, decode_tokens, mutation=None, max_len=40):
    """Prompt logits, the hidden states of greedy-decode steps fed with
    decode_tokens, and every layer's K / V rows for all positions."""
    f = Float64Llama(m, max_len, mutation)
    for t, tok in enumerate(prompt):
        f.step(int(tok), t)
    logits = f.logits()
    hids = [f.step(int(tok), len(prompt) + i).copy() for i, tok in enumerate(decode_tokens)]
    n = len(prompt) + len(decode_tokens)
    kv = [(f.K[l, :n].reshape(n, -1), f.V[l, :n].reshape(n, -1)) for l in range(len(f.layers))]
    return logits, hids, kv


def run_oracle(m, prompt, n_decode=4, max_len=40):
    o = ref.Llama(m, max_len)
    tok, logits = o.prefill(prompt)
    toks, hids = [], []
    for i in range(n_decode):
        toks.append(tok)
        tok, hid = o.decode(tok, len(prompt) + i)
        hids.append(hid)
    n = len(prompt) + n_decode
    kv = [(ref.f16_to_f32(o.kcache(l, max_len)[:n]), ref.f16_to_f32(o.vcache(l, max_len)[:n]))
          for l in range(m["config"]["n_layers"])]
    return logits, toks, hids, kv


def errors(oracle_run, f64_run):
    """(worst per-layer K/V relative error, worst logits / hidden error)"""
    logits, _, hids, kv = oracle_run
    f_logits, f_hids, f_kv = f64_run
    kv_err = max(max(rel(k, fk), rel(v, fv)) for (k, v), (fk, fv) in zip(kv, f_kv))
    out_err = max([rel(logits, f_logits)] + [rel(h, fh) for h, fh in zip(hids, f_hids)])
    return kv_err, out_err


def applicable(mutation, cfg):
    """gqa_modulo is the same map when every query head has its own kv
    head or all share one."""
    kvmul = cfg["n_heads"] // cfg["n_kv_heads"]
    return mutation != "gqa_modulo" or (kvmul > 1 and cfg["n_kv_heads"] > 1)


@pytest.fixture(scope="module")
def cases(oracle_lib):
    out = []
    for i, kw in enumerate(CONFIGS):
        m = sensitive_llama(**kw)
        prompt = np.random.default_rng(100 + i).integers(0, m["config"]["vocab"], 14)
        out.append((m, prompt, run_oracle(m, prompt)))
    return out


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_oracle_llama_matches_float64_forward(cases, ci):
    """Every layer's K / V cache rows (prefill and four decode steps), the
    prompt's last logits and the decode steps' hidden states of the oracle's
    decoder equal the float64 textbook forward within KV_TOL / OUT_TOL."""
    m, prompt, orun = cases[ci]
    frun = run_float64(m, prompt, orun[1])
    kv_err, out_err = errors(orun, frun)
    assert kv_err < KV_TOL, kv_err
    assert out_err < OUT_TOL, out_err


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_float64_forward_sees_each_composition_mistake(cases, mutation):
    """Each planted mistake moves the float64 forward away from the oracle by
    more than 3x the tolerance (in the K / V rows or in the outputs) on every
    config where it changes the function, so the agreement above would fail
    had the oracle made that mistake."""
    scores = []
    for m, prompt, orun in cases:
        if not applicable(mutation, m["config"]):
            continue
        kv_err, out_err = errors(orun, run_float64(m, prompt, orun[1], mutation))
        scores.append(max(kv_err / KV_TOL, out_err / OUT_TOL))
    assert scores and min(scores) > 3.0, (mutation, scores)


def _cache_view(o, layer, which, max_len):
    kvd = o.cfg["n_kv_heads"] * o.cfg["head_dim"]
    fn = ref.lib().ref_llama_kcache if which == "k" else ref.lib().ref_llama_vcache
    ptr = fn(o.state, layer)
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint16)), (max_len, kvd))


def test_oracle_ignores_cache_rows_past_position(oracle_lib):
    """Causality: garbage written into every KV row past the decode position
    (all layers, K and V) leaves the decode step's output bit-identical."""
    m = sensitive_llama(**CONFIGS[0])
    prompt = np.random.default_rng(7).integers(0, m["config"]["vocab"], 9)
    max_len = 32
    clean, dirty = ref.Llama(m, max_len), ref.Llama(m, max_len)
    ta, _ = clean.prefill(prompt)
    tb, _ = dirty.prefill(prompt)
    pos = len(prompt)
    rng = np.random.default_rng(8)
    for l in range(m["config"]["n_layers"]):
        for which in "kv":
            view = _cache_view(dirty, l, which, max_len)
            view[pos:] = rng.integers(0, 0x7bff, view[pos:].shape, dtype=np.uint16)
    a, ha = clean.decode(ta, pos)
    b, hb = dirty.decode(tb, pos)
    assert a == b and np.array_equal(ha.view(np.uint32), hb.view(np.uint32))


def test_oracle_zero_wo_w2_leaves_normed_embedding(oracle_lib):
    """Residual wiring: with wo and w2 all zero (zero blocks decode to 0, so
    both projections add exactly 0), the output-normed hidden state is
    rmsnorm(embedding row, out_norm) for every position."""
    m = sensitive_llama(**CONFIGS[0])
    c = m["config"]
    zero_wo = np.zeros((c["dim"], c["n_heads"] * c["head_dim"]), np.float32)
    zero_w2 = np.zeros((c["dim"], c["hidden"]), np.float32)
    m["wo"] = [ref.quantize_rows(c["layer_type"], zero_wo)] * c["n_layers"]
    m["w2"] = [ref.quantize_rows(c["layer_type"], zero_w2)] * c["n_layers"]
    o = ref.Llama(m, 16)
    emb = ref.dequant(ref.Q4_K, m["tok_embd"], c["vocab"], c["dim"])
    tok = 5
    for pos in range(4):
        nxt, hid = o.decode(tok, pos)
        want = ref.rmsnorm(emb[tok], m["out_norm"], c["rms_eps"])
        assert np.array_equal(hid.view(np.uint32), want.view(np.uint32)), pos
        # and against the textbook norm in float64
        x = emb[tok].astype(np.float64)
        tb = x / np.sqrt(np.mean(x * x) + c["rms_eps"]) * m["out_norm"]
        assert np.allclose(hid, tb, rtol=2e-6, atol=1e-7)
        tok = nxt


def test_oracle_gqa_map_commutes_with_kv_head_renumbering(oracle_lib):
    """GQA map: renumber the kv heads by a permutation (rows of wk / wv) and
    move each head's query group with it (rows of wq, columns of wo).  With
    query head h reading kv head h / kvMul the model is the same function:
    every K / V row is the same row at its new head, and every logit agrees
    to float rounding (each wo row dot then sums the same Q8K blocks in
    another order).  A modulo map pairs query groups with other kv heads and
    is a different function.  A query group here is 2 x 128 = 256 columns,
    one super-block, so the permutation moves whole encoded blocks of wo and
    whole Q8K blocks of the attention output: the permuted model holds the
    same bytes."""
    kw = dict(CONFIGS[0])
    kw.update(n_heads=8, n_kv_heads=4, head_dim=128, dim=512)
    m = sensitive_llama(**kw)
    c = m["config"]
    hd, kvmul, nkv, lt = c["head_dim"], c["n_heads"] // c["n_kv_heads"], c["n_kv_heads"], c["layer_type"]
    perm = np.array([2, 0, 3, 1])  # new kv head g is old kv head perm[g]
    dim, qd = c["dim"], c["n_heads"] * hd
    rb_in, rb_q = ref.row_bytes(lt, dim), ref.row_bytes(lt, qd)
    gblk = kvmul * hd // 256  # encoded blocks per query group in a wo row
    bb = rb_q // (qd // 256)
    m2 = dict(m)
    for name in ("wq", "wk", "wv", "wo"):
        m2[name] = []
    for l in range(c["n_layers"]):
        wq = m["wq"][l].reshape(qd, rb_in)
        wk = m["wk"][l].reshape(nkv * hd, rb_in)
        wv = m["wv"][l].reshape(nkv * hd, rb_in)
        wo = m["wo"][l].reshape(dim, qd // 256, bb)
        krows = np.concatenate([np.arange(perm[g] * hd, (perm[g] + 1) * hd) for g in range(nkv)])
        qrows = np.concatenate([np.arange(perm[g] * kvmul * hd, (perm[g] + 1) * kvmul * hd)
                                for g in range(nkv)])
        oblk = np.concatenate([np.arange(perm[g] * gblk, (perm[g] + 1) * gblk) for g in range(nkv)])
        m2["wq"].append(np.ascontiguousarray(wq[qrows]).reshape(-1))
        m2["wk"].append(np.ascontiguousarray(wk[krows]).reshape(-1))
        m2["wv"].append(np.ascontiguousarray(wv[krows]).reshape(-1))
        m2["wo"].append(np.ascontiguousarray(wo[:, oblk]).reshape(-1))
    prompt = np.random.default_rng(9).integers(0, c["vocab"], 10)
    a, b = ref.Llama(m, 16), ref.Llama(m2, 16)
    a.prefill(prompt)
    b.prefill(prompt)

    def rows(o, l, which):
        h = o.kcache(l, 16) if which == "k" else o.vcache(l, 16)
        return ref.f16_to_f32(h[:10]).reshape(10, nkv, hd)

    # layer 0's K / V rows see only the embedding: exactly the old rows moved
    for which in "kv":
        assert np.array_equal(rows(b, 0, which), rows(a, 0, which)[:, perm])
    # layer 1's rows see layer 0's attention through wo.  They agree to
    # float rounding (measured 1e-3: the reordered wo sums, then Q8K), while
    # a modulo query-to-kv map moves them by O(1) (0.77 in the float64
    # forward on CONFIGS[0]).  The last logits are not compared: peaked
    # attention turns single Q8K rounding flips into percent-level drift.
    for which in "kv":
        assert rel(rows(b, 1, which), rows(a, 1, which)[:, perm]) < 1e-2
    f_ok = Float64Llama(m, 16)
    f_bad = Float64Llama(m, 16, mutation="gqa_modulo")
    for t, tok in enumerate(prompt):
        f_ok.step(int(tok), t)
        f_bad.step(int(tok), t)
    assert rel(f_bad.K[1, :10], f_ok.K[1, :10]) > 0.1


def test_rope_dot_depends_only_on_relative_position(oracle_lib):
    """q.k after the oracle's interleaved RoPE depends on the position
    difference only: rope(q, p + d) . rope(k, p' + d) == rope(q, p) . rope(k,
    p') to float rounding, while the unrotated dot differs."""
    hd = 64
    inv = ref.rope_inv_freq(500000.0, hd)
    q, k = normal(1, hd), normal(2, hd)

    def rot(v, pos):
        s, c = ref.rope_sincos(pos, inv)
        return ref.rope_apply(v, hd, 1, s, c).astype(np.float64)

    base = rot(q, 7) @ rot(k, 3)
    for d in (1, 50, 400):
        assert abs(rot(q, 7 + d) @ rot(k, 3 + d) - base) < 2e-5 * np.abs(q).sum()
    assert abs(rot(q, 7) @ rot(k, 7) - rot(q, 7) @ rot(k, 3)) > 1e-2


def test_oracle_decode_resumes_from_copied_cache(oracle_lib):
    """set_kv: a second state whose cache rows 0..P-1 are copied from a state
    that ran the prompt decodes the same tokens and hidden states from
    position P (the benchmark's CPU baseline starts decoding that way)."""
    m = sensitive_llama(**CONFIGS[0])
    prompt = np.random.default_rng(9).integers(0, m["config"]["vocab"], 11)
    max_len, P = 24, len(prompt)
    src, dst = ref.Llama(m, max_len), ref.Llama(m, max_len)
    tok, _ = src.prefill(prompt)
    for l in range(m["config"]["n_layers"]):
        dst.set_kv(l, 0, src.kcache(l, max_len)[:P], src.vcache(l, max_len)[:P])
    ta = tb = tok
    for i in range(5):
        ta, ha = src.decode(ta, P + i)
        tb, hb = dst.decode(tb, P + i)
        assert ta == tb and np.array_equal(ha.view(np.uint32), hb.view(np.uint32)), i
    with pytest.raises(AssertionError):
        dst.set_kv(0, max_len - 2, src.kcache(0, max_len)[:3], src.vcache(0, max_len)[:3])
