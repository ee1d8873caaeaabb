"""Oracle pins for the row-dot formats beyond Q4_K / Q6_K / Q8_0: Q5_K, Q4_0,
Q4_1, MXFP4, Q2_K and Q3_K (kernels_amd64.s:550-1128, quant_q8k_portable.go:
132-390).

* The amd64-order restatement agrees with the independently written portable
  restatement within the reference's own bar, 1e-3 * (1 + |want|), on the
  patterns the reference's tests use: random rows at 256..4096 columns, the
  all-0xff extremes with +-1 activations, the lane-order byte patterns, the
  Q3_K hmask extremes and every MXFP4 code (q5k_q8_amd64_test.go,
  q4_01_q8_amd64_test.go, mxfp4_q8_amd64_test.go, q2k_q8_amd64_test.go,
  q3k_q8_amd64_test.go).
* The per-lane integers equal a numpy decoding of the block layouts
  (DequantRow*Into's code extraction) dotted with the same q8, lane by lane.
* The int8 path stays close to the float path through the dequantised rows
  (TestQ*Q8MatvecCloseToFloat): cosine >= 0.999.
"""
import numpy as np
import pytest

from conftest import BLOCK, extreme_row, f16b, normal, random_rows
from oracle import oracle as ref

def prepared(qtype, x):
    cols = x.size
    q8 = np.empty(cols, np.int8)
    xsc = np.empty(cols // 256, np.float32)
    ref.lib().ref_q8k_quantize(ref._p(ref._f32(x)), ref._p(q8), ref._p(xsc), cols // 256)
    if qtype in (ref.Q5_K, ref.Q4_0, ref.Q4_1):
        xs = ref.xsums32(x)
    elif qtype == ref.Q2_K:
        xs = ref.xsums16(x, scale32=False)
    else:
        xs = None
    return q8, xsc, xs


def close(got, want):
    return abs(got - want) <= 1e-3 * (1 + abs(want))


def both_orders(qtype, row, x):
    q8, xsc, xs = prepared(qtype, x)
    a = ref.row_dot(qtype, row, q8, xsc, xs, ref.AMD64)
    g = ref.row_dot(qtype, row, q8, xsc, xs, ref.GENERIC)
    return a, g


# --------------------------------------------------- numpy block decoders --
def codes_and_scales(qtype, row, cols):
    """(integer code per element, integer weight per element) such that the
    lane integer is sum(weight * code * q8) over the lane's elements; weight
    is the sub-block scale where the format folds one in."""
    bb, be = BLOCK[qtype]
    blk = np.asarray(row, np.uint8).reshape(-1, bb).astype(np.int64)
    n = blk.shape[0]
    e = np.arange(be)
    if qtype == ref.Q5_K:
        s, l = (e % 64) // 32 + 0, e % 32          # s: low(0)/high(1) half of chunk
        chunk = e // 64
        q = blk[:, 48 + chunk * 32 + l]
        nib = np.where(s == 0, q & 15, q >> 4)
        bit = (blk[:, 16 + l] >> (2 * chunk + s)) & 1
        code = nib | (bit << 4)
        sc = np.zeros((n, 8), np.int64)
        for j in range(8):
            sb = blk[:, 4:16]
            if j < 4:
                sc[:, j] = sb[:, j] & 63
            else:
                sc[:, j] = (sb[:, j + 4] & 15) | ((sb[:, j - 4] >> 6) << 4)
        weight = sc[:, e // 32]
    elif qtype in (ref.Q4_0, ref.Q4_1):
        off = 2 if qtype == ref.Q4_0 else 4
        byte = blk[:, off + (e % 16)]
        code = np.where(e < 16, byte & 15, byte >> 4)
        weight = np.ones_like(code)
    elif qtype == ref.MXFP4:
        dbl = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12])
        byte = blk[:, e // 2]
        code = dbl[np.where(e % 2 == 0, byte & 15, byte >> 4)]
        weight = np.ones_like(code)
    elif qtype == ref.Q2_K:
        m = e // 32
        code = (blk[:, 16 + 32 * (m // 4) + e % 32] >> (2 * (m % 4))) & 3
        weight = blk[:, e // 16] & 15
    else:  # Q3_K
        m = e // 32
        u = (blk[:, 32 + 32 * (m // 4) + e % 32] >> (2 * (m % 4))) & 3
        h = (blk[:, e % 32] >> m) & 1
        code = u - 4 * (1 - h)
        a0 = blk[:, 96:100] @ (256 ** np.arange(4))
        a1 = blk[:, 100:104] @ (256 ** np.arange(4))
        t = blk[:, 104:108] @ (256 ** np.arange(4))
        aux = [(a0 & 0x0f0f0f0f) | ((t & 0x03030303) << 4),
               (a1 & 0x0f0f0f0f) | (((t >> 2) & 0x03030303) << 4),
               ((a0 >> 4) & 0x0f0f0f0f) | (((t >> 4) & 0x03030303) << 4),
               ((a1 >> 4) & 0x0f0f0f0f) | (((t >> 6) & 0x03030303) << 4)]
        sc = np.stack([(aux[i // 4] >> (8 * (i % 4))) & 0xff for i in range(16)], 1)
        weight = sc[:, e // 16] - 32
    return code.reshape(-1, 256), weight.reshape(-1, 256)


@pytest.mark.parametrize("qtype", list(BLOCK))
def test_lane_ints_match_numpy_decoding(oracle_lib, qtype):
    cols = 1024
    row = random_rows(qtype, 1, cols, 11 + qtype)
    q8, _, _ = prepared(qtype, normal(12, cols))
    got = ref.lane_ints(qtype, row, q8)                     # [blocks][8]
    code, w = codes_and_scales(qtype, row, cols)
    prod = (code * w * q8.astype(np.int64).reshape(-1, 256))
    # lane k of 32-element group m holds elements 32m + 4k .. 32m + 4k + 3
    want = prod.reshape(-1, 8, 8, 4).sum(axis=(1, 3))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("qtype", list(BLOCK))
@pytest.mark.parametrize("cols", [256, 512, 1024, 4096])
def test_amd64_order_matches_portable(oracle_lib, qtype, cols):
    """Tests *DotQ8KRowMatchesReference: random rows, N(0, 1) activations."""
    for s in range(3):
        row = random_rows(qtype, 1, cols, 100 * qtype + cols + s)
        a, g = both_orders(qtype, row, normal(7 + s, cols))
        assert close(a, g), (a, g)


@pytest.mark.parametrize("qtype", list(BLOCK))
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_extremes(oracle_lib, qtype, sign):
    """TestAudit*DotExtremes: every code byte 0xff, d (and dmin / m) 1,
    x = +-1 (q8 = +-127).  Closed forms per 256 elements at x = +1:
    Q5_K 63*31*256 - 63*32*8, Q2_K 15*3*256 - 15*16*16, Q3_K (63-32)*3*256,
    Q4_0 (15-8)*256, Q4_1 15*256 + 32*8, MXFP4 -6*256."""
    cols = 1024
    row = extreme_row(qtype, cols)
    x = np.full(cols, sign, np.float32)
    a, g = both_orders(qtype, row, x)
    assert close(a, g), (a, g)
    per = {ref.Q5_K: 63 * 31 * 256 - 63 * 32 * 8, ref.Q2_K: 15 * 3 * 256 - 15 * 16 * 16,
           ref.Q3_K: 31 * 3 * 256, ref.Q4_0: 7 * 256, ref.Q4_1: 15 * 256 + 32 * 8,
           ref.MXFP4: -6 * 256}[qtype]
    assert np.isclose(a, sign * per * cols / 256, rtol=1e-5), (a, sign * per * cols / 256)


@pytest.mark.parametrize("qtype", list(BLOCK))
def test_lane_order_pattern(oracle_lib, qtype):
    """TestAudit*DotLaneOrder: byte (i*53 + b*29) & 0xff, small scales,
    x = ((i % 97) - 48) / 48."""
    cols = 512
    bb, be = BLOCK[qtype]
    nb = cols // be
    i = np.arange(bb)
    blk = np.stack([((i * 53 + b * 29) & 0xFF) for b in range(nb)]).astype(np.uint8)
    ref_row = extreme_row(qtype, cols).reshape(nb, bb)
    hdr = {ref.Q5_K: [0, 1, 2, 3], ref.Q4_0: [0, 1], ref.Q4_1: [0, 1, 2, 3], ref.MXFP4: [],
           ref.Q2_K: [80, 81, 82, 83], ref.Q3_K: [108, 109]}[qtype]
    blk[:, hdr] = ref_row[:, hdr]
    if qtype in (ref.Q5_K, ref.Q4_1, ref.Q2_K):
        lo = 2 if qtype != ref.Q2_K else 82
        blk[:, lo:lo + 2] = f16b(1 / 256)  # dmin / m small, as the reference's 0x3000
    if qtype == ref.MXFP4:
        blk[:, 16] = 120 + np.arange(nb) % 8
    x = (((np.arange(cols) % 97) - 48) / 48).astype(np.float32)
    a, g = both_orders(qtype, blk.reshape(-1), x)
    assert close(a, g), (a, g)


@pytest.mark.parametrize("fill", [0x00, 0xFF, 0x55])
def test_q3k_hmask_extremes(oracle_lib, fill):
    """TestQ3KDotQ8KRowAsmHmaskExtremes / striped hmask: every high bit
    set (no element biased), none set (all biased by -4), alternating."""
    cols = 512
    row = random_rows(ref.Q3_K, 1, cols, 61).reshape(-1, 110)
    row[:, 0:32] = fill
    a, g = both_orders(ref.Q3_K, row.reshape(-1), normal(62, cols))
    assert close(a, g), (a, g)


def test_q3k_scale_bias_and_unpack(oracle_lib):
    """TestQ3KDotQ8KRowAsmScaleBiasAndUnpack: one block, every scale value,
    codes 3 with the high bit set (value 3), x = 1: result = 3 * sum(dl) * 16 / 127 * 127."""
    for sc in (0, 1, 31, 32, 33, 63):
        blk = np.zeros(110, np.uint8)
        blk[0:32] = 0xFF
        blk[32:96] = 0xFF
        lo, hi = sc & 15, sc >> 4
        blk[96:104] = lo | (lo << 4)
        blk[104:108] = hi | (hi << 2) | (hi << 4) | (hi << 6)
        blk[108:110] = f16b(1.0)
        x = np.ones(256, np.float32)
        a, g = both_orders(ref.Q3_K, blk, x)
        assert close(a, g)
        assert np.isclose(a, 3 * (sc - 32) * 256, rtol=1e-5), (sc, a)


def test_mxfp4_all_codes(oracle_lib):
    """TestAuditMXFP4DotAllCodes: every code 0..15 in every position."""
    cols = 1024
    nb = cols // 32
    blk = np.zeros((nb, 17), np.uint8)
    for b in range(nb):
        for i in range(16):
            blk[b, i] = ((2 * i + b) & 15) | (((2 * i + 1 + b) & 15) << 4)
        blk[b, 16] = 127
    for sign in (1.0, -1.0):
        x = np.full(cols, sign, np.float32)
        a, g = both_orders(ref.MXFP4, blk.reshape(-1), x)
        assert close(a, g)


@pytest.mark.parametrize("qtype", list(BLOCK))
def test_int8_path_close_to_float(oracle_lib, qtype):
    """TestQ*Q8MatvecCloseToFloat: the int8-activation matvec against the
    dequantised rows dotted in float64."""
    rows, cols = 64, 1024
    data = random_rows(qtype, rows, cols, 80 + qtype)
    x = normal(81, cols)
    got = ref.matvec(qtype, data, x, rows, cols)
    w = np.stack([ref.dequant_row(qtype, data[r * ref.row_bytes(qtype, cols):
                                              (r + 1) * ref.row_bytes(qtype, cols)], cols)
                  for r in range(rows)]).astype(np.float64)
    want = w @ x.astype(np.float64)
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    assert cos >= 0.999, cos
