"""Greedy token identity on the full synthetic Llama-3-8B-shape model
32 layers, d = 4096, ffn 14336, 32/8 GQA heads of
128, vocab 128256; Q4_K attention/FFN and token embedding, Q6_K output head,
RMSNorm weights 1.0, weights N(0, 0.02) generated on the device.  A 512-token
uniform-random prompt is prefilled and 128 tokens are decoded greedily on the
GPU; the CPU oracle (AVX2 port of kernels_amd64.s, bit-identical to the
lane-level restatement) runs the same weights, downloaded in GGUF layout.
"""
import time

import numpy as np
import pytest

from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def test_llama3_8b_shape_greedy_identical_to_oracle(hip):
    from gopherllm_amd import synth

    if not ref.has_avx2():
        pytest.skip("host lacks AVX2 for the full-size oracle run")
    cfg = dict(synth.LLAMA3_8B)
    prompt_len, n_gen = 512, 128
    t0 = time.time()
    gpu = synth.build_decoder(cfg, max_len=prompt_len + n_gen, seed=1)
    prompt = np.random.default_rng(2024).integers(0, cfg["vocab"], prompt_len)
    first, logits = gpu.prefill(prompt, want_logits=True)
    # a meaningful comparison needs live logits: N(0, ~1.3^2) for this model
    assert np.isfinite(logits).all(), "non-finite prefill logits"
    assert 0.5 < float(np.std(logits)) < 5.0, float(np.std(logits))
    assert first == int(np.argmax(logits))
    got = [first]
    for i in range(1, n_gen):
        got.append(gpu.decode(got[-1], prompt_len + i - 1))
    got = np.array(got, np.uint32)
    assert len(set(got.tolist())) > 8, f"degenerate greedy output {got[:16]}"
    t1 = time.time()
    m = synth.host_model(gpu)
    gpu.release()
    cpu = ref.Llama(m, prompt_len + n_gen, fast=True)
    want = cpu.generate(prompt, n_gen)
    t2 = time.time()
    print(f"8B greedy: GPU build+generate {t1 - t0:.1f} s, CPU oracle {t2 - t1:.1f} s; "
          f"first tokens {got[:8].tolist()}", flush=True)
    diff = np.flatnonzero(got != want)
    assert diff.size == 0, f"tokens differ from position {diff[0]}: {got[diff[0]:diff[0] + 4]} vs " \
                           f"{want[diff[0]:diff[0] + 4]}"
