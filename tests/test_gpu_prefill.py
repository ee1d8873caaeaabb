"""Batched prefill products on the matrix cores.

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


def amd64(data, xs, rows, cols):
    want = ref.matvec_batch_fast(ref.Q4_K, data, xs, rows, cols)
    if want is None:
        want = ref.matvec_batch(ref.Q4_K, data, xs, rows, cols)
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


@pytest.mark.parametrize("rows", [4096, 14336])
def test_prefill_configs2(hip, rows):
    """Q4_K rows x 4096 (seeded N(0, 0.02), device RTN encoder)
    against 512 activation rows N(0, 1)."""
    import torch
    cols, p = 4096, 512
    tmp = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    hip.fill_normal_dev(tmp, 3000 + rows, 0.02)
    raw = torch.empty(rows * hip.row_bytes(hip.TYPE_Q4_K, cols), dtype=torch.uint8, device="cuda")
    hip.quantize_rows_dev(hip.TYPE_Q4_K, tmp, raw)
    w = hip.Weight.from_device(raw, hip.TYPE_Q4_K, rows, cols)
    del tmp
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
    sel = [0, 1, 31, 32, 100, 255, 256, 511]
    xh = x.cpu().numpy()[sel]
    want = amd64(raw.cpu().numpy(), xh, rows, cols)
    assert_bits(got[sel], want, "sampled tokens vs amd64 oracle")
