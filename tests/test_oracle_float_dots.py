"""Oracle pins for the float-activation row dots of the reference's same-type
fused groups (matvecSameType2/3Into via sameTypeQuantDot, model.go:3213-3283):
DotQ8_0F32 (simd.go:646), DotQ4_0F32 (simd.go:677), DotQ4_1F32
(quant_extra.go:42), DotQ2KF32 (quant_extra.go:271), DotQ3KF32
(quant_extra.go:376), DotQ5KF32 (simd.go:1031) and DotMXFP4F32
(simd.go:1458).

* Every dot agrees with the dequantised row dotted in float64 within the
  reference's own bar, 1e-3 * (1 + |want|) (TestDotQ8_0F32MatchesNaiveDequant,
  TestExtraQuantDotMatchesDequantizedDot).
* The accumulation order is pinned by inputs whose float32 result depends on
  it: one element of 2**24 followed in the same accumulator by elements of 1
  absorbs them (2**24 + 1 rounds to 2**24, ties to even), while 1s that
  reach a different accumulator, or that are summed before the large
  element, survive.  Each case's expected value follows from which elements
  share an accumulator and in which order; a single sequential accumulator, a
  different lane split or a reversed order gives another value.
"""
import numpy as np
import pytest

from conftest import BLOCK, f16b, random_rows
from oracle import oracle as ref

FLOAT_TYPES = (ref.Q8_0, ref.Q4_0, ref.Q4_1, ref.Q2_K, ref.Q3_K, ref.Q5_K, ref.MXFP4)
BIG = np.float32(2.0 ** 24)


def rows_of(qtype, rows, cols, seed):
    if qtype == ref.Q8_0:
        w = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.02).astype(np.float32)
        return ref.quantize_rows(ref.Q8_0, w)
    return random_rows(qtype, rows, cols, seed)


@pytest.mark.parametrize("qtype", FLOAT_TYPES)
@pytest.mark.parametrize("cols", [256, 1024, 4096])
def test_float_dot_matches_float64_dequant(oracle_lib, qtype, cols):
    rows = 8
    data = rows_of(qtype, rows, cols, 90 + qtype)
    x = np.random.default_rng(91).standard_normal(cols).astype(np.float32)
    got = ref.matvec_float(qtype, data, x, rows, cols)
    rb = ref.row_bytes(qtype, cols)
    for r in range(rows):
        w = ref.dequant_row(qtype, data[r * rb:(r + 1) * rb], cols).astype(np.float64)
        want = float(w @ x.astype(np.float64))
        assert abs(got[r] - want) <= 1e-3 * (1 + abs(want)), (qtype, cols, r, got[r], want)
        assert got[r] == np.float32(ref.float_dot(qtype, data[r * rb:(r + 1) * rb], x, cols))


def q8_0_block(codes, d=1.0):
    return np.concatenate([f16b(d), np.asarray(codes, np.int8).view(np.uint8)])


def test_q8_0_order():
    """s_j accumulates elements j, 4+j, ..., 28+j in order; the four lanes
    meet only in (s0 + s1) + (s2 + s3)."""
    codes = np.zeros(32, np.int8)
    codes[[0, 4, 8]] = 1
    x = np.zeros(32, np.float32)
    x[0], x[4], x[8] = BIG, 1, 1
    # s0 = ((2^24 + 1) + 1) = 2^24: the 1s follow the large element
    assert ref.float_dot(ref.Q8_0, q8_0_block(codes), x, 32) == BIG
    codes[:] = 0
    codes[[0, 1, 5]] = 1
    x[:] = 0
    x[0], x[1], x[5] = BIG, 1, 1
    # s0 = 2^24, s1 = 2 (elements 1 and 5 share lane 1): 2^24 + 2 is exact
    assert ref.float_dot(ref.Q8_0, q8_0_block(codes), x, 32) == BIG + 2
    # the scale multiplies the lane sum once: 3 * (2^24 + 2)
    assert ref.float_dot(ref.Q8_0, q8_0_block(codes, 3.0), x, 32) == np.float32(3) * (BIG + 2)


def q4_block(lo, hi, d=1.0, m=None):
    """nibble codes (0..15) of elements 0..15 (lo) and 16..31 (hi)"""
    packed = (np.asarray(lo, np.uint8) & 15) | ((np.asarray(hi, np.uint8) & 15) << 4)
    head = f16b(d) if m is None else np.concatenate([f16b(d), f16b(m)])
    return np.concatenate([head, packed])


def test_q4_0_order():
    """s_j += (lo * x[i+j] + hi * x[16+i+j]) for i = 0, 4, 8, 12: the pair is
    summed first, codes are nibble - 8."""
    lo, hi = np.full(16, 8), np.full(16, 8)   # code 0 everywhere
    lo[0], hi[0], lo[4] = 9, 9, 9             # +1 at elements 0, 16, 4
    x = np.zeros(32, np.float32)
    x[0], x[16], x[4] = BIG, 1, 1
    # pair (0, 16) = 2^24 + 1 -> 2^24; then lane 0 adds element 4: 2^24
    assert ref.float_dot(ref.Q4_0, q4_block(lo, hi), x, 32) == BIG
    lo[0], hi[0], lo[4], lo[1] = 9, 8, 8, 9   # +1 at elements 0 and 1 only
    x[:] = 0
    x[0], x[1] = BIG, 2
    # lanes 0 and 1 meet in (s0 + s1): 2^24 + 2
    assert ref.float_dot(ref.Q4_0, q4_block(lo, hi), x, 32) == BIG + 2
    lo[:] = 8
    hi[:] = 8
    lo[0] = 0                                  # code -8
    x[:] = 0
    x[0] = 1
    assert ref.float_dot(ref.Q4_0, q4_block(lo, hi, 0.5), x, 32) == -4


def test_q4_1_order():
    """qdot += (lo*x[i] + hi*x[16+i]) and xsum += (x[i] + x[16+i]) in i
    order, then d*qdot + m*xsum."""
    lo, hi = np.zeros(16), np.zeros(16)
    lo[0], hi[0], lo[1] = 1, 1, 1
    x = np.zeros(32, np.float32)
    x[0], x[16], x[1] = BIG, 1, 1
    # qdot: (2^24 + 1) -> 2^24, + (1 + 0) -> 2^24;
    # xsum: (2^24 + 1) -> 2^24, + (1 + 0) -> 2^24; d = 1, m = 1: 2^25
    assert ref.float_dot(ref.Q4_1, q4_block(lo, hi, 1.0, 1.0), x, 32) == 2 * BIG
    # m = 0 keeps the qdot term alone; m = -1 cancels it exactly
    assert ref.float_dot(ref.Q4_1, q4_block(lo, hi, 1.0, 0.0), x, 32) == BIG
    assert ref.float_dot(ref.Q4_1, q4_block(lo, hi, 1.0, -1.0), x, 32) == 0


def k_block(qtype, scale_nibbles, codes, d=1.0, dmin=0.0):
    """A Q2_K / Q3_K block: 16 sub-block scales, per-element 2-bit codes
    (Q3_K: hmask bits all set, so values are the codes), d (and dmin)."""
    codes = np.asarray(codes, np.int64)
    qs = np.zeros(64, np.uint8)
    for e in range(256):
        m = e // 32
        qs[32 * (m // 4) + e % 32] |= (codes[e] & 3) << (2 * (m % 4))
    if qtype == ref.Q2_K:
        sc = np.asarray(scale_nibbles, np.uint8) & 15
        return np.concatenate([sc, qs, f16b(d), f16b(dmin)])
    # Q3_K: scales 6-bit biased by 32, packed as in q3KScales (low nibbles in
    # bytes 0..7, high 2 bits in bytes 8..11)
    s6 = (np.asarray(scale_nibbles, np.int64) + 32) & 63
    packed = np.zeros(12, np.uint8)
    for i in range(16):
        lo4, hi2 = s6[i] & 15, s6[i] >> 4
        packed[i % 8] |= lo4 << (4 * (i // 8))
        packed[8 + i % 4] |= hi2 << (2 * (i // 4))
    hmask = np.full(32, 0xff, np.uint8)
    return np.concatenate([hmask, qs, packed, f16b(d)])


@pytest.mark.parametrize("qtype", [ref.Q2_K, ref.Q3_K])
def test_k_float_dot_order(qtype):
    """Per 16-element sub-block an in-order sum, then the sub-block terms are
    added to the row sum in sub-block order."""
    codes = np.zeros(256, np.int64)
    codes[[0, 1, 2]] = 1
    scales = np.zeros(16, np.int64)
    scales[0] = 1
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2] = BIG, 1, 1
    blk = k_block(qtype, scales, codes)
    # sub-block 0: ((2^24 + 1) + 1) -> 2^24, times d * scale = 1
    assert ref.float_dot(qtype, blk, x, 256) == BIG
    # two sub-blocks: 2^24 from sub-block 0, then + 2 (sub-block 1: 1 + 1)
    codes[:] = 0
    codes[[0, 16, 17]] = 1
    scales[1] = 1
    x[:] = 0
    x[0], x[16], x[17] = BIG, 1, 1
    assert ref.float_dot(qtype, k_block(qtype, scales, codes), x, 256) == BIG + 2


def test_q3k_hmask_and_q2k_min():
    # Q3_K: a clear hmask bit subtracts 4 from the code
    codes = np.zeros(256, np.int64)
    codes[0] = 3
    scales = np.zeros(16, np.int64)
    scales[0] = 1
    blk = k_block(ref.Q3_K, scales, codes)
    blk[0] = 0xfe   # element 0's bit (bit 0 of hmask byte 0) cleared
    x = np.zeros(256, np.float32)
    x[0] = 1
    assert ref.float_dot(ref.Q3_K, blk, x, 256) == -1
    # Q2_K: sum += dl*qdot - ml*xsum, min nibble in the high half
    sc = np.zeros(16, np.int64)
    sc[0] = 0x21    # scale 1, min 2
    blk = k_block(ref.Q2_K, sc, np.zeros(256), 1.0, 0.5)
    blk[0] = 0x21
    x[:] = 0
    x[0], x[1] = 3, 5
    assert ref.float_dot(ref.Q2_K, blk, x, 256) == -(1.0 * 8)   # 0 - (0.5*2)*(3+5)


def test_mxfp4_order():
    """sum += (lut[code] * scale) * x element by element across the row."""
    blk = np.zeros(17, np.uint8)
    blk[0] = 0x22      # elements 0, 1: 1.0
    blk[1] = 0x02      # element 2: 1.0
    blk[16] = 127      # scale 1
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = BIG, 1, 1
    assert ref.float_dot(ref.MXFP4, blk, x, 32) == BIG
    x[:] = 0
    x[1], x[2], x[0] = 1, 1, BIG
    blk[16] = 128      # scale 2: lut*scale first, exact
    assert ref.float_dot(ref.MXFP4, blk, x, 32) == 2 * BIG


def q5k_block(codes, sc, m, d=1.0, dmin=0.0):
    """A Q5_K block from 5-bit codes per element and 6-bit scales / mins per
    32-element sub-block (scaleMinK4 packing, simd.go:1524-1528)."""
    codes = np.asarray(codes, np.int64)
    scales = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            scales[j] |= sc[j] & 63
            scales[j + 4] |= m[j] & 63
        else:
            scales[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
            scales[j - 4] |= (sc[j] >> 4) << 6
            scales[j] |= (m[j] >> 4) << 6
    qh, q = np.zeros(32, np.uint8), np.zeros(128, np.uint8)
    for e in range(256):
        st, half, l = e // 64, (e // 32) % 2, e % 32
        q[32 * st + l] |= (codes[e] & 15) << (4 * half)
        qh[l] |= (codes[e] >> 4) << (2 * st + half)
    return np.concatenate([f16b(d), f16b(dmin), scales, qh, q])


def test_q5k_order():
    """Four lane accumulators (element l % 4) per 32-element half, joined as
    (a0 + a1) + (a2 + a3); each half's d1*qdot - min1*xsum is added to the
    row sum in half order."""
    sc, m = np.zeros(8, np.int64), np.zeros(8, np.int64)
    sc[:3] = 1
    codes = np.zeros(256, np.int64)
    codes[[0, 4, 8]] = 1
    x = np.zeros(256, np.float32)
    x[0], x[4], x[8] = BIG, 1, 1
    assert ref.float_dot(ref.Q5_K, q5k_block(codes, sc, m), x, 256) == BIG
    codes[:] = 0
    codes[[0, 1, 5]] = 1
    x[:] = 0
    x[0], x[1], x[5] = BIG, 1, 1
    assert ref.float_dot(ref.Q5_K, q5k_block(codes, sc, m), x, 256) == BIG + 2
    # halves 0, 1, 2 each add their own term: (2^24 + 1) + 1 = 2^24, where
    # adding the two later halves first would give 2^24 + 2
    codes[:] = 0
    codes[[0, 32, 64]] = 1
    x[:] = 0
    x[0], x[32], x[64] = BIG, 1, 1
    assert ref.float_dot(ref.Q5_K, q5k_block(codes, sc, m), x, 256) == BIG
    # the high bit adds 16 to the nibble; the min term subtracts
    # dmin * m * xsum: 16 * 1 - (0.5 * 2) * (1 + 3)
    codes[:] = 0
    codes[0] = 16
    m[0] = 2
    x[:] = 0
    x[0], x[1] = 1, 3
    assert ref.float_dot(ref.Q5_K, q5k_block(codes, sc, m, 1.0, 0.5), x, 256) == 16 - 4
    # sub-blocks 4..7 take the split 6-bit packing: scale 33 in sub-block 5
    sc[:] = 0
    m[:] = 0
    sc[5] = 33
    codes[:] = 0
    codes[5 * 32 + 3] = 1
    x[:] = 0
    x[5 * 32 + 3] = 1
    assert ref.float_dot(ref.Q5_K, q5k_block(codes, sc, m), x, 256) == 33
