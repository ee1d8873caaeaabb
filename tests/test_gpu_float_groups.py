"""GPU parity of the decode-step fused groups that the reference runs through
its float kernels (matvecSameType2/3Into via sameTypeQuantDot,
model.go:3213-3283: DotQ8_0F32, DotQ4_0F32, DotQ4_1F32, DotQ2KF32, DotQ3KF32,
DotQ5KF32, DotMXFP4F32), of the routing of mixed groups
(tryMatvecAttentionInto / tryMatvec2Into, model.go:3157-3206), of
Weight.RowInto (model.go:1034-1100) for every weight type, and of resident
llama decoders whose layers and embeddings are in those formats: bit for bit
against the oracle, through the C ABI."""
import numpy as np
import pytest

from conftest import normal, quant_matrix, tiny_llama
from oracle import oracle as ref

pytestmark = pytest.mark.gpu

FLOAT_TYPES = (ref.Q8_0, ref.Q4_0, ref.Q4_1, ref.Q2_K, ref.Q3_K, ref.Q5_K, ref.MXFP4)
NAME = {ref.F32: "f32", ref.F16: "f16", ref.BF16: "bf16", ref.Q8_0: "q8_0", ref.Q4_0: "q4_0",
        ref.Q4_1: "q4_1", ref.Q2_K: "q2k", ref.Q3_K: "q3k", ref.Q4_K: "q4k", ref.Q5_K: "q5k",
        ref.Q6_K: "q6k", ref.MXFP4: "mxfp4"}


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_bits(got, want, what):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.flatnonzero(bits(got).ravel() != bits(want).ravel())
    assert bad.size == 0, f"{what}: {bad.size} values differ, first {bad[:4]}: " \
        f"{got.ravel()[bad[:4]]} vs {want.ravel()[bad[:4]]}"


def weight(hip, qtype, rows, cols, seed):
    data, _ = quant_matrix(qtype, rows, cols, seed)
    return data, hip.Weight.from_host(data, qtype, rows, cols)


@pytest.mark.parametrize("qtype", FLOAT_TYPES, ids=[NAME[t] for t in FLOAT_TYPES])
@pytest.mark.parametrize("rows,cols", [(37, 256), (300, 1024), (1024, 4096), (40, 14336)])
def test_same_type_groups_bit_exact(hip, qtype, rows, cols):
    """A same-type pair and triple: every output is the float kernel's."""
    shapes = (rows, rows + 5, rows // 2 + 1)
    ws = [weight(hip, qtype, r, cols, 10 * i + rows + cols + qtype) for i, r in enumerate(shapes)]
    x = normal(rows + cols, cols)
    x[100:140] = 0.0
    want = [ref.matvec_float(qtype, d, x, r, cols) for (d, _), r in zip(ws, shapes)]
    print(f"float group {NAME[qtype]} {rows}x{cols}", flush=True)
    oa, ob = hip.matvec2_into(ws[0][1], ws[1][1], x)
    assert_bits(oa, want[0], "pair a")
    assert_bits(ob, want[1], "pair b")
    outs = hip.matvec3_into(ws[0][1], ws[1][1], ws[2][1], x)
    for i in range(3):
        assert_bits(outs[i], want[i], f"triple {i}")


@pytest.mark.parametrize("qtype", FLOAT_TYPES, ids=[NAME[t] for t in FLOAT_TYPES])
def test_device_group_entry_and_batches(hip, qtype):
    """gllm_hip_matvec_multi_dev: batch 1 is the fused group (float kernels),
    batches run matvecBatchQ8's int8 row dots per weight."""
    import torch
    rows, cols = 200, 2048
    ws = [weight(hip, qtype, rows + 3 * i, cols, 50 + i + qtype) for i in range(3)]
    for p in (1, 5):
        xs = normal(60 + p, (p, cols))
        outs = [torch.empty((p, w.rows), dtype=torch.float32, device="cuda") for _, w in ws]
        hip.matvec_multi_dev([w for _, w in ws], torch.from_numpy(xs).cuda(), outs)
        torch.cuda.synchronize()
        for (d, w), o in zip(ws, outs):
            want = (ref.matvec_float(qtype, d, xs[0], w.rows, cols) if p == 1
                    else ref.matvec_batch(qtype, d, xs, w.rows, cols))
            assert_bits(o.cpu().numpy().reshape(p, -1), np.asarray(want).reshape(p, -1), f"p={p}")


MIXED = [
    ((ref.Q8_0, ref.Q8_0, ref.Q6_K), (1, 1, 0)),   # pair (0, 1) fused, 2 on its own
    ((ref.Q8_0, ref.Q4_K, ref.Q8_0), (1, 0, 1)),   # pair (0, 2)
    ((ref.Q4_K, ref.Q4_0, ref.Q4_0), (0, 1, 1)),   # pair (1, 2)
    ((ref.Q4_K, ref.Q4_K, ref.Q6_K), (0, 0, 0)),   # MatvecQ4K2Q6KIntoWithXSums
    ((ref.Q6_K, ref.Q6_K, ref.Q6_K), (0, 0, 0)),   # MatvecQ6K3Into
    ((ref.Q4_0, ref.Q8_0, ref.Q5_K), (0, 0, 0)),   # no pair: three MatvecInto
    ((ref.Q4_K, ref.Q8_0, ref.Q4_K), (0, 0, 0)),   # Q4_K pair: int8
]


@pytest.mark.parametrize("types,floats", MIXED, ids=["-".join(NAME[t] for t in ty)
                                                     for ty, _ in MIXED])
def test_mixed_triples_route_as_the_reference(hip, types, floats):
    rows, cols = 130, 1024
    ws = [weight(hip, t, rows + i, cols, 70 + 7 * i + t) for i, t in enumerate(types)]
    x = normal(71, cols)
    outs = hip.matvec3_into(*[w for _, w in ws], x)
    for i, ((d, w), t, fl) in enumerate(zip(ws, types, floats)):
        want = ref.matvec_float(t, d, x, w.rows, cols) if fl else ref.matvec(t, d, x, w.rows, cols)
        assert_bits(outs[i], want, f"weight {i} ({NAME[t]}, {'float' if fl else 'int8'})")


def test_mixed_pair_runs_int8(hip):
    """A pair of two formats is not fused: each runs its own MatvecInto."""
    rows, cols = 90, 512
    (da, wa), (db, wb) = weight(hip, ref.Q4_0, rows, cols, 81), weight(hip, ref.Q8_0, rows, cols, 82)
    x = normal(83, cols)
    oa, ob = hip.matvec2_into(wa, wb, x)
    assert_bits(oa, ref.matvec(ref.Q4_0, da, x, rows, cols), "q4_0")
    assert_bits(ob, ref.matvec(ref.Q8_0, db, x, rows, cols), "q8_0")


ROW_TYPES = (ref.F32, ref.F16, ref.BF16, ref.Q8_0, ref.Q4_0, ref.Q4_1, ref.Q2_K, ref.Q3_K,
             ref.Q4_K, ref.Q5_K, ref.Q6_K, ref.MXFP4)


@pytest.mark.parametrize("qtype", ROW_TYPES, ids=[NAME[t] for t in ROW_TYPES])
def test_weight_rows_bit_exact(hip, qtype):
    """gllm_hip_weight_rows_dev == DequantRow*Into / rawScalarRowInto of each
    requested row, repeated and out-of-order ids included."""
    import torch
    rows, cols = 301, 768
    data, _ = quant_matrix(qtype, rows, cols, 90 + qtype)
    if qtype == ref.F16:
        # every f16 class: subnormals, infinities, NaNs with payloads
        h = data.view(np.uint16).copy()
        h[:6] = [0x0001, 0x03ff, 0x7c00, 0xfc00, 0x7c01, 0xfe00]
        data = h.view(np.uint8)
    w = hip.Weight.from_host(data, qtype, rows, cols)
    ids = np.array([0, 300, 5, 5, 177, 1, 299], np.uint32)
    out = torch.empty((ids.size, cols), dtype=torch.float32, device="cuda")
    w.rows_dev(torch.from_numpy(ids.view(np.int32)).cuda(), out)
    torch.cuda.synchronize()
    rb = ref.row_bytes(qtype, cols)
    want = np.stack([ref.dequant_row(qtype, data[i * rb:(i + 1) * rb], cols) for i in ids])
    assert_bits(out.cpu().numpy(), want, NAME[qtype])


def test_scalar_weights_have_no_row_kernel(hip):
    data, _ = quant_matrix(ref.F16, 8, 256, 3)
    w = hip.Weight.from_host(data, ref.F16, 8, 256)
    with pytest.raises(hip.GllmError):
        w.matvec_into(np.ones(256, np.float32))


def decode_matches(hip, m, prompt, n_steps, max_len):
    from gopherllm_amd.decoder import LlamaDecoder
    gpu = LlamaDecoder.from_host_model(m, max_len)
    cpu = ref.Llama(m, max_len)
    gt, gl = gpu.prefill(prompt, want_logits=True)
    ct, cl = cpu.prefill(prompt)
    assert_bits(gl, cl, "prefill logits")
    assert gt == ct
    tok = ct
    for pos in range(len(prompt), len(prompt) + n_steps):
        want, hid = cpu.decode(tok, pos)
        got = gpu.decode(tok, pos)
        assert_bits(gpu.hidden(), hid, f"hidden at {pos}")
        assert got == want, pos
        tok = want


def test_q8_0_llama_decodes_with_the_oracle(hip):
    """A Q8_0 file (every matrix and the embeddings): prompt tokens take the
    int8 row dots per matrix, generation steps the float kernels for Q/K/V
    and gate/up, the int8 row dots for the output, down and vocabulary
    projections."""
    m = tiny_llama(seed=21, n_layers=2, dim=512, hidden=1024, n_heads=8, n_kv_heads=2,
                   head_dim=64, vocab=900, layer_type=ref.Q8_0, out_type=ref.Q8_0,
                   emb_type=ref.Q8_0)
    prompt = np.random.default_rng(22).integers(0, 900, 20)
    print("q8_0 llama", flush=True)
    decode_matches(hip, m, prompt, 10, 64)


MIX = {"wq": ref.Q4_0, "wk": ref.Q4_0, "wv": ref.Q8_0, "wo": ref.Q3_K, "w1": ref.Q5_K,
       "w2": ref.Q2_K, "w3": ref.Q5_K}


@pytest.mark.parametrize("emb", [ref.F16, ref.BF16, ref.F32, ref.Q6_K, ref.MXFP4],
                         ids=["f16", "bf16", "f32", "q6k", "mxfp4"])
def test_mixed_format_llama_decodes_with_the_oracle(hip, emb):
    """Q4_0 Q/K pair (float) with a Q8_0 V (int8), Q5_K gate/up (float),
    Q3_K output and Q2_K down projections, and embeddings of another type."""
    m = tiny_llama(seed=23, n_layers=2, dim=256, hidden=512, n_heads=4, n_kv_heads=2,
                   head_dim=64, vocab=700, out_type=ref.Q4_1, emb_type=emb,
                   type_of=lambda l, k: MIX[k])
    prompt = np.random.default_rng(24).integers(0, 700, 12)
    print(f"mixed-format llama, embeddings {NAME[emb]}", flush=True)
    decode_matches(hip, m, prompt, 6, 48)


def test_output_without_row_kernel_rejected(hip):
    """An F16 output projection (the reference's raw scalar matvec) has no
    row kernel here: decode refuses the model instead of computing it
    another way."""
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=25, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1,
                   head_dim=64, vocab=300, out_type=ref.F16)
    gpu = LlamaDecoder.from_host_model(m, 32)
    with pytest.raises(hip.GllmError):
        gpu.decode(1, 0)


@pytest.mark.parametrize("qtype", [ref.Q4_K, ref.Q8_0, ref.Q5_K], ids=["q4k", "q8_0", "q5k"])
@pytest.mark.parametrize("dim,hidden", [(256, 512), (4096, 14336)])
def test_swiglu_down_path(hip, qtype, dim, hidden):
    """gllm_hip_swiglu_down_dev == down.MatvecInto(siluMulF32(gate, up)) with
    gate / up from the fused pair (int8 for Q4_K, the float kernels for the
    other formats) and down's own int8 row dot."""
    import torch
    (dg, wg), (du, wu) = (weight(hip, qtype, hidden, dim, 100 + i) for i in range(2))
    dd, wd = weight(hip, qtype, dim, hidden, 102)
    x = normal(103, dim)
    out = torch.empty(dim, dtype=torch.float32, device="cuda")
    hip.swiglu_down_dev(wg, wu, wd, torch.from_numpy(x).cuda(), out)
    torch.cuda.synchronize()
    mv = ref.matvec if qtype == ref.Q4_K else ref.matvec_float
    h = ref.silu_mul(mv(qtype, dg, x, hidden, dim), mv(qtype, du, x, hidden, dim))
    assert_bits(out.cpu().numpy(), ref.matvec(qtype, dd, h, dim, hidden), "swiglu down")
