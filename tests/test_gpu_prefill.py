"""Batched prefill products: Q4_K and Q6_K on the matrix cores,
Q8_0 on 64 x 64 tiles of the vector units.

matvecBatchQ8 (kernels_amd64.go:470-581) evaluates q4kDotQ8KRow once per
(row, token), so the batched result must equal the per-token row kernel bit
for bit: checked against the amd64-order oracle on small shapes (ragged row
and token tiles, degenerate activation blocks) and, at the configs[2] sizes,
against the oracle on sampled tokens plus the GPU's own batch-1 path on every
token (the reference's batched == per-token invariant, forward_batch_test.go).
"""
import numpy as np
import pytest

from conftest import normal, quant_matrix
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def amd64(data, xs, rows, cols, qtype=ref.Q4_K):
    want = ref.matvec_batch_fast(qtype, data, xs, rows, cols)
    if want is None:
        want = ref.matvec_batch(qtype, data, xs, rows, cols)
    return want.reshape(xs.shape[0], rows)


def assert_bits(got, want, what):
    bad = np.argwhere(bits(got) != bits(want))
    assert bad.size == 0, f"{what}: {len(bad)} values differ, first (token, row) {bad[:4].tolist()}: " \
        f"{got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"


@pytest.mark.parametrize("rows,cols,p", [(300, 1024, 16), (300, 1024, 33), (64, 256, 100),
                                         (1000, 4096, 64), (70, 14336, 40)])
def test_prefill_bit_exact_small(hip, rows, cols, p):
    data, _ = quant_matrix(ref.Q4_K, rows, cols, 500 + p + rows)
    w = hip.Weight.from_host(data, ref.Q4_K, rows, cols)
    xs = normal(501 + p, (p, cols))
    print(f"prefill {rows}x{cols} p={p}", flush=True)
    got = w.matvec_batch(xs)
    assert_bits(got, amd64(data, xs, rows, cols), "vs amd64 oracle")


def test_prefill_degenerate_blocks(hip):
    """All-zero tokens, zero 256-blocks inside a token, a lone large value and
    NaN-free extremes (q8kQuantize's scale-0 blocks, quant_q8k_portable.go:36-62)."""
    rows, cols, p = 130, 1024, 20
    data, _ = quant_matrix(ref.Q4_K, rows, cols, 77)
    w = hip.Weight.from_host(data, ref.Q4_K, rows, cols)
    xs = normal(78, (p, cols))
    xs[0] = 0.0
    xs[3, 256:512] = 0.0
    xs[5, :] = 0.0
    xs[5, 700] = -3.5
    xs[7] *= 1e4
    xs[9] = np.float32(1e-30)
    got = w.matvec_batch(xs)
    assert_bits(got, amd64(data, xs, rows, cols), "degenerate activations")


def test_prefill_extremes_closed_form(hip):
    """TestAuditQ4KDotExtremes (q4k_q8_amd64_audit_test.go:18-52) batched: every
    code byte 0xff, d = dmin = 1, x = +-1 -> q8 = +-127, sc = m = 63, nibbles 15;
    per block 63 * 15 * 127 * 256 - 63 * 32 * 8 (x = +1)."""
    rows, cols, p = 48, 1024, 32
    blk = np.full(144, 0xFF, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    data = np.tile(blk, rows * (cols // 256))
    w = hip.Weight.from_host(data, ref.Q4_K, rows, cols)
    xs = np.where(np.arange(p)[:, None] % 2 == 0, 1.0, -1.0).astype(np.float32) * np.ones((p, cols),
                                                                                          np.float32)
    got = w.matvec_batch(xs)
    # the integer parts are exact; d * xscale = 1/127 rounds, hence rtol
    per_block = 63.0 * 15 * 256 - 63.0 * 32 * 8
    assert np.allclose(got[0::2], per_block * (cols // 256), rtol=1e-6)
    assert np.allclose(got[1::2], -per_block * (cols // 256), rtol=1e-6)
    assert_bits(got, amd64(data, xs, rows, cols), "extremes")


def device_weight(hip, qtype, rows, cols, seed):
    """Seeded N(0, 0.02) rows encoded on the device (the RTN encoders)."""
    import torch
    tmp = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    hip.fill_normal_dev(tmp, seed, 0.02)
    raw = torch.empty(rows * hip.row_bytes(qtype, cols), dtype=torch.uint8, device="cuda")
    hip.quantize_rows_dev(qtype, tmp, raw)
    del tmp
    return hip.Weight.from_device(raw, qtype, rows, cols), raw


@pytest.mark.parametrize("rows", [4096, 14336])
def test_prefill_configs2(hip, rows):
    """Q4_K rows x 4096 (seeded N(0, 0.02), device RTN encoder)
    against 512 activation rows N(0, 1): every token against the amd64-order
    oracle and against the GPU's own batch-1 path."""
    import torch
    cols, p = 4096, 512
    w, raw = device_weight(hip, hip.TYPE_Q4_K, rows, cols, 3000 + rows)
    x = torch.empty((p, cols), dtype=torch.float32, device="cuda")
    hip.fill_normal_dev(x, 77, 1.0)
    out = torch.empty((p, rows), dtype=torch.float32, device="cuda")
    print(f"prefill configs[2] {rows}x{cols} p={p}", flush=True)
    w.matvec_dev(x, out)
    one = torch.empty((p, rows), dtype=torch.float32, device="cuda")
    for t in range(p):
        w.matvec_dev(x[t:t + 1], one[t:t + 1])
    torch.cuda.synchronize()
    got, per_token = out.cpu().numpy(), one.cpu().numpy()
    assert np.isfinite(got).all() and float(np.std(got)) > 0.1
    assert_bits(got, per_token, "batched vs per-token row kernel")
    want = amd64(raw.cpu().numpy(), x.cpu().numpy(), rows, cols)
    assert_bits(got, want, "every token vs amd64 oracle")


# Q6_K batches of more than 16 tokens take the matrix-core tiles when the
# row has a multiple of 8 blocks (2048 columns and up); 1024 columns keep the
# row kernels (same bits either way)
@pytest.mark.parametrize("rows,cols,p", [(300, 2048, 17), (300, 2048, 33), (64, 2048, 100),
                                         (1000, 4096, 64), (70, 14336, 40), (130, 1024, 40)])
def test_prefill_q6k_bit_exact_small(hip, rows, cols, p):
    data, _ = quant_matrix(ref.Q6_K, rows, cols, 600 + p + rows)
    w = hip.Weight.from_host(data, ref.Q6_K, rows, cols)
    xs = normal(601 + p, (p, cols))
    print(f"prefill Q6_K {rows}x{cols} p={p}", flush=True)
    got = w.matvec_batch(xs)
    assert_bits(got, amd64(data, xs, rows, cols, ref.Q6_K), "vs amd64 oracle")


def test_prefill_q6k_extremes(hip):
    """Scales -128 and 127 with codes 63 (the largest |sc * code|, past f16's
    exact integers: the split at the code's fields keeps it exact), zero and
    large activations, against the oracle."""
    rows, cols, p = 64, 2048, 24
    rng = np.random.default_rng(91)
    data, _ = quant_matrix(ref.Q6_K, rows, cols, 92)
    blocks = data.reshape(rows * (cols // 256), 210)
    blocks[0::2, 0:192] = 0xFF                  # every code 63
    blocks[0::2, 192:208] = np.where(rng.random((len(blocks[0::2]), 16)) < 0.5, 0x80, 0x7F)
    blocks[1::4, 192:208] = 0x80                # scale -128 with random codes
    xs = normal(93, (p, cols))
    xs[0] = 0.0
    xs[1] *= 1e4
    xs[2, :] = np.where(np.arange(cols) % 2 == 0, 1.0, -1.0)
    w = hip.Weight.from_host(data, ref.Q6_K, rows, cols)
    got = w.matvec_batch(xs)
    assert_bits(got, amd64(data, xs, rows, cols, ref.Q6_K), "extremes vs amd64 oracle")


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_prefill_q6k_configs2_shapes(hip, rows, cols):
    """Q6_K at the configs[1] / configs[2] shapes (a Q4_K_M file's ffn_down
    and attn_v are Q6_K), 512 tokens: every token against the amd64-order
    oracle."""
    import torch
    p = 512
    w, raw = device_weight(hip, hip.TYPE_Q6_K, rows, cols, 4000 + rows)
    x = torch.empty((p, cols), dtype=torch.float32, device="cuda")
    hip.fill_normal_dev(x, 78, 1.0)
    out = torch.empty((p, rows), dtype=torch.float32, device="cuda")
    print(f"prefill Q6_K {rows}x{cols} p={p}", flush=True)
    w.matvec_dev(x, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all() and float(np.std(got)) > 0.1
    want = amd64(raw.cpu().numpy(), x.cpu().numpy(), rows, cols, ref.Q6_K)
    assert_bits(got, want, "every token vs amd64 oracle")


@pytest.mark.parametrize("rows,cols,p", [(300, 1024, 17), (64, 256, 100), (1000, 4096, 64),
                                         (70, 14336, 40), (130, 2048, 33)])
def test_prefill_q8_0_bit_exact_small(hip, rows, cols, p):
    """Q8_0 batches of more than 16 tokens (64 x 64 tiles on the vector
    units): ragged row and token tiles against the amd64-order oracle."""
    data, _ = quant_matrix(ref.Q8_0, rows, cols, 700 + p + rows)
    w = hip.Weight.from_host(data, ref.Q8_0, rows, cols)
    xs = normal(701 + p, (p, cols))
    xs[0] = 0.0
    xs[1] *= 1e4
    print(f"prefill Q8_0 {rows}x{cols} p={p}", flush=True)
    got = w.matvec_batch(xs)
    assert_bits(got, amd64(data, xs, rows, cols, ref.Q8_0), "vs amd64 oracle")


def test_prefill_q8_0_extremes(hip):
    """Weights -128 and 127 against activations +-127: every 4-byte dot at
    its extremes (the reference's VPMADDUBSW pairs stay inside int16)."""
    rows, cols, p = 64, 1024, 20
    data, _ = quant_matrix(ref.Q8_0, rows, cols, 94)
    blocks = data.reshape(rows * (cols // 32), 34)
    blocks[0::2, 2:] = 0x80                     # -128
    blocks[1::2, 2:] = 0x7F                     # 127
    xs = np.where(np.arange(cols) % 3 == 0, 1.0, -1.0).astype(np.float32) * np.ones((p, 1), np.float32)
    xs[1::2] *= -1.0
    w = hip.Weight.from_host(data, ref.Q8_0, rows, cols)
    got = w.matvec_batch(xs)
    assert_bits(got, amd64(data, xs, rows, cols, ref.Q8_0), "extremes vs amd64 oracle")


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_prefill_q8_0_configs2_shapes(hip, rows, cols):
    """Q8_0 at the configs[1] / configs[2] shapes, 512 tokens: every token
    against the amd64-order oracle."""
    import torch
    p = 512
    w, raw = device_weight(hip, hip.TYPE_Q8_0, rows, cols, 5000 + rows)
    x = torch.empty((p, cols), dtype=torch.float32, device="cuda")
    hip.fill_normal_dev(x, 79, 1.0)
    out = torch.empty((p, rows), dtype=torch.float32, device="cuda")
    print(f"prefill Q8_0 {rows}x{cols} p={p}", flush=True)
    w.matvec_dev(x, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all() and float(np.std(got)) > 0.1
    want = amd64(raw.cpu().numpy(), x.cpu().numpy(), rows, cols, ref.Q8_0)
    assert_bits(got, want, "every token vs amd64 oracle")
