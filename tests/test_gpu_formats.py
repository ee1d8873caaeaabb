"""GPU parity of the Q5_K, Q4_0, Q4_1, MXFP4, Q2_K and Q3_K row kernels: bit
for bit against the amd64-order oracle (kernels_amd64.s:550-1128) through the
C ABI, at batch 1 and in batches, with 1, 2 and 4 lanes per AVX2 lane (the
shapes choose them), ragged row counts, the all-0xff extremes and the
upload repack's inverse; and, for these formats, Q6_K and Q8_0, the batch-1
kernels that quantise x themselves against the same kernels fed by the
separate quantiser launch."""
import numpy as np
import pytest

from conftest import BLOCK, NAMES, extreme_row, normal, quant_matrix, random_rows
from oracle import oracle as ref

pytestmark = pytest.mark.gpu

FORMATS = list(BLOCK)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_bits(got, want, what):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.flatnonzero(bits(got).ravel() != bits(want).ravel())
    assert bad.size == 0, f"{what}: {bad.size} values differ, first {bad[:4]}: " \
        f"{got.ravel()[bad[:4]]} vs {want.ravel()[bad[:4]]}"


@pytest.mark.parametrize("qtype", FORMATS, ids=[NAMES[q] for q in FORMATS])
@pytest.mark.parametrize("rows,cols", [(1, 256), (37, 512), (37, 768), (21, 2304), (300, 1024),
                                       (1000, 4096), (4096, 4096), (600, 14336)])
def test_matvec_bit_exact(hip, qtype, rows, cols):
    data = random_rows(qtype, rows, cols, rows + cols + qtype)
    x = normal(rows * 3 + cols, cols)
    x[300:340] = 0.0
    w = hip.Weight.from_host(data, qtype, rows, cols)
    print(f"format {NAMES[qtype]} {rows}x{cols}", flush=True)
    assert_bits(w.matvec_into(x), ref.matvec(qtype, data, x, rows, cols), "batch 1")


@pytest.mark.parametrize("qtype", FORMATS, ids=[NAMES[q] for q in FORMATS])
@pytest.mark.parametrize("rows,cols", [(37, 512), (37, 768), (300, 1024), (4096, 4096)])
def test_batches_bit_exact(hip, qtype, rows, cols):
    """matvecBatchQ8 == per-token row kernel, for 4- and 8-token tiles."""
    data = random_rows(qtype, rows, cols, 7 * rows + qtype)
    w = hip.Weight.from_host(data, qtype, rows, cols)
    for p in (3, 8, 13):
        xs = normal(p + rows, (p, cols))
        print(f"format {NAMES[qtype]} {rows}x{cols} p={p}", flush=True)
        got = w.matvec_batch(xs)
        assert_bits(got, ref.matvec_batch(qtype, data, xs, rows, cols), f"p={p}")


@pytest.mark.parametrize("qtype", FORMATS, ids=[NAMES[q] for q in FORMATS])
def test_extremes_and_degenerate_activations(hip, qtype):
    cols, rows = 1024, 40
    data = np.tile(extreme_row(qtype, cols), rows)
    w = hip.Weight.from_host(data, qtype, rows, cols)
    for x in (np.ones(cols, np.float32), -np.ones(cols, np.float32), np.zeros(cols, np.float32)):
        assert_bits(w.matvec_into(x), ref.matvec(qtype, data, x, rows, cols), "extremes")
    rnd = random_rows(qtype, rows, cols, 90 + qtype)
    w2 = hip.Weight.from_host(rnd, qtype, rows, cols)
    x = normal(91, cols)
    x[:256] = 0.0
    x[700] = 1e4
    assert_bits(w2.matvec_into(x), ref.matvec(qtype, rnd, x, rows, cols), "degenerate")


@pytest.mark.parametrize("qtype", FORMATS, ids=[NAMES[q] for q in FORMATS])
def test_download_roundtrip_and_argmax(hip, qtype):
    import torch
    rows, cols = 333, 512
    data = random_rows(qtype, rows, cols, 55 + qtype)
    w = hip.Weight.from_host(data, qtype, rows, cols)
    out = torch.empty(data.size, dtype=torch.uint8, device="cuda")
    w.download_dev(out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), data)
    x = normal(56, cols)
    assert w.argmax_matvec(x) == ref.argmax_finite(ref.matvec(qtype, data, x, rows, cols))


def test_fused_pair_of_other_types_runs_float_kernel(hip):
    """matvecSameType2Into (model.go:3213-3230) runs DotQ5KF32 for a Q5_K
    pair: both outputs are the float kernel's, not the int8 row dot's."""
    data = random_rows(ref.Q5_K, 64, 256, 1)
    a = hip.Weight.from_host(data, ref.Q5_K, 64, 256)
    x = normal(2, 256)
    oa, ob = hip.matvec2_into(a, a, x)
    want = ref.matvec_float(ref.Q5_K, data, x, 64, 256)
    assert_bits(oa, want, "pair a")
    assert_bits(ob, want, "pair b")


@pytest.mark.parametrize("qtype", [ref.Q6_K, ref.Q8_0] + FORMATS,
                         ids=["q6k", "q8_0"] + [NAMES[q] for q in FORMATS])
@pytest.mark.parametrize("rows,cols", [(37, 512), (37, 768), (1000, 4096), (4100, 4096)])
def test_fused_quantisation_matches_prequantised(hip, qtype, rows, cols):
    """At batch 1 with cols <= 4096 the row kernels quantise x in LDS
    themselves; the same kernels fed by the separate Q8K-prep launch
    (gllm_hip_q8k_prepare_dev + gllm_hip_matvec_q8_dev) and the oracle agree
    bit for bit, ragged last workgroup included."""
    import torch
    if qtype in BLOCK:
        data = random_rows(qtype, rows, cols, 3 * rows + qtype)
    else:
        data, _ = quant_matrix(qtype, rows, cols, 5 * rows + qtype)
    x = normal(rows + 17, cols)
    x[100:140] = 0.0
    w = hip.Weight.from_host(data, qtype, rows, cols)
    print(f"fused vs prequantised type {qtype} {rows}x{cols}", flush=True)
    fused = w.matvec_into(x)
    xd = torch.from_numpy(x).cuda()
    act = torch.empty(hip.act_bytes(cols, 1), dtype=torch.uint8, device="cuda")
    hip.q8k_prepare_dev(xd, act)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    w.matvec_q8_dev(act, 1, out)
    torch.cuda.synchronize()
    want = ref.matvec(qtype, data, x, rows, cols)
    assert_bits(fused, want, "fused")
    assert_bits(out.cpu().numpy(), want, "prequantised")
