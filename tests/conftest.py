"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU.

Synthetic data: numpy PCG64 streams from fixed seeds (the reference's own
tests use Go math/rand, which cannot be regenerated here).  Weights are
N(0, 0.02) quantised with the oracle's restatement of the reference RTN
encoders; activations N(0, 1).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as ref  # noqa: E402  (checker only)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def normal(seed, shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std)
            ).astype(np.float32)


def quant_matrix(qtype, rows, cols, seed, std=0.02):
    """GGUF-layout bytes of a rows x cols matrix of type qtype: N(0, std)
    values quantised by the oracle (Q4_K, Q6_K, Q8_0), stored as they are
    (F32, F16, BF16 truncated), or random codes with sane scales for the
    other block formats (random_rows)."""
    w = normal(seed, (rows, cols), std)
    if qtype == ref.F32:
        return w.view(np.uint8).reshape(-1), w
    if qtype == ref.F16:
        return w.astype(np.float16).view(np.uint8).reshape(-1), w
    if qtype == ref.BF16:
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1), w
    if qtype in BLOCK:
        return random_rows(qtype, rows, cols, seed), w
    return ref.quantize_rows(qtype, w), w


MATRICES = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


def tiny_llama(seed=1, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2, head_dim=64,
               vocab=1000, layer_type=ref.Q4_K, out_type=ref.Q6_K, type_of=None,
               emb_type=ref.Q4_K):
    """A small llama-shaped model with the reference's tensor roles
    (model.go:2027 loadLayer) and RMSNorm weights of 1.0.  type_of(layer,
    name), if given, picks each matrix's type (mixed files such as Q4_K_M)
    and the model then carries "types" [n_layers][7] in MATRICES order."""
    cfg = dict(n_layers=n_layers, dim=dim, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv_heads,
               head_dim=head_dim, vocab=vocab, rms_eps=1e-5, rope_theta=500000.0,
               emb_type=emb_type, out_type=out_type, layer_type=layer_type)
    qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
    s = seed * 1000
    m = {"config": cfg}
    m["tok_embd"], _ = quant_matrix(emb_type, vocab, dim, s + 1)
    m["output"], _ = quant_matrix(out_type, vocab, dim, s + 2)
    m["out_norm"] = np.ones(dim, np.float32)
    shapes = {"wq": (qd, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, qd),
              "w1": (hidden, dim), "w2": (dim, hidden), "w3": (hidden, dim)}
    tof = type_of or (lambda l, k: layer_type)
    for k, (r, c) in shapes.items():
        m[k] = [quant_matrix(tof(l, k), r, c, s + 10 + 10 * l + list(shapes).index(k))[0]
                for l in range(n_layers)]
    if type_of is not None:
        m["types"] = [[int(tof(l, k)) for k in MATRICES] for l in range(n_layers)]
    m["attn_norm"] = [np.ones(dim, np.float32) for _ in range(n_layers)]
    m["ffn_norm"] = [np.ones(dim, np.float32) for _ in range(n_layers)]
    return m


def q4km_types(l, name):
    """Q4_K_M-style mix for tiny_llama(type_of=...): attn_v and ffn_down in
    Q6_K on every other layer, the rest Q4_K."""
    return ref.Q6_K if name in ("wv", "w2") and l % 2 == 0 else ref.Q4_K


@pytest.fixture(scope="session")
def oracle_lib():
    ref.build()
    return ref.lib()


@pytest.fixture(scope="session")
def hip():
    """The product library on a gfx950 device; skips when no GPU is present
    (CPU runs), fails loudly if the library is missing on a GPU box."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gopherllm_amd as g
    g.load()
    if not g.available():
        pytest.fail("libgllm_hip loaded but no gfx950 device: " + g._lib.last_error())
    return g


# ---- rows of the formats beyond Q4_K / Q6_K / Q8_0 ----------------------
BLOCK = {ref.Q5_K: (176, 256), ref.Q4_0: (18, 32), ref.Q4_1: (20, 32), ref.MXFP4: (17, 32),
         ref.Q2_K: (84, 256), ref.Q3_K: (110, 256)}
NAMES = {ref.Q5_K: "q5k", ref.Q4_0: "q4_0", ref.Q4_1: "q4_1", ref.MXFP4: "mxfp4",
         ref.Q2_K: "q2k", ref.Q3_K: "q3k"}


def f16b(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def random_rows(qtype, rows, cols, seed):
    """Random codes with sane scales (the reference's randomQ*Row helpers)."""
    rng = np.random.default_rng(seed)
    bb, be = BLOCK[qtype]
    nb = rows * cols // be
    blk = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    d = rng.uniform(0.002, 0.02, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    m = rng.uniform(0.001, 0.01, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if qtype == ref.Q5_K:
        blk[:, 0:2], blk[:, 2:4] = d, m
    elif qtype == ref.Q4_0:
        blk[:, 0:2] = d
    elif qtype == ref.Q4_1:
        blk[:, 0:2], blk[:, 2:4] = d, m
    elif qtype == ref.MXFP4:
        blk[:, 16] = rng.integers(118, 130, nb)
    elif qtype == ref.Q2_K:
        blk[:, 80:82], blk[:, 82:84] = d, m
    elif qtype == ref.Q3_K:
        blk[:, 108:110] = d
    return blk.reshape(-1)


def extreme_row(qtype, cols):
    bb, be = BLOCK[qtype]
    blk = np.full((cols // be, bb), 0xFF, np.uint8)
    one = f16b(1.0)
    if qtype == ref.Q5_K:
        blk[:, 0:2], blk[:, 2:4] = one, one
    elif qtype == ref.Q4_0:
        blk[:, 0:2] = one
    elif qtype == ref.Q4_1:
        blk[:, 0:2], blk[:, 2:4] = one, one
    elif qtype == ref.MXFP4:
        blk[:, 16] = 127
    elif qtype == ref.Q2_K:
        blk[:, 80:82], blk[:, 82:84] = one, one
    elif qtype == ref.Q3_K:
        blk[:, 108:110] = one
    return blk.reshape(-1)
