"""The load-time known-answer check in gopherllm_amd/csrc/gemv.hip
(self_check) expects exact integers from the matvec path.  These CPU tests
rebuild its inputs byte for byte and show that the oracle's amd64-order
restatement of the row kernels (kernels_amd64.s:437-543, 1123-1220,
1321-1391) returns exactly those integers, so a device that passes the
check agrees with the reference on these inputs, and the check cannot fail
on a correct device for lack of float exactness."""
import numpy as np
import pytest

from oracle import oracle as ref

ROWS = 8192
CASES = [(ref.Q4_K, 1024, 3), (ref.Q6_K, 512, 1), (ref.Q8_0, 1024, 3)]


def check_inputs(qtype, cols, xr):
    rb = ref.row_bytes(qtype, cols)
    bb = rb // (cols // 256)
    i = np.arange(rb, dtype=np.int64)
    r = np.arange(ROWS, dtype=np.int64)[:, None]
    w = ((i[None, :] * (7 + 6 * r + qtype) + 3 * r + 1) & 0xFF).astype(np.uint8)
    for b in range(cols // 256):
        if qtype == ref.Q4_K:
            w[:, b * bb:b * bb + 4] = [0x00, 0x3C, 0x00, 0x3C]  # d = dmin = 1.0
        elif qtype == ref.Q6_K:
            w[:, b * bb + 208:b * bb + 210] = [0x00, 0x3C]
        else:
            for j in range(8):
                w[:, b * bb + 34 * j:b * bb + 34 * j + 2] = [0x00, 0x3C]
    x = (((np.arange(cols) * 37 + 11) % (2 * xr + 1)) - xr).astype(np.float32)
    for b in range(cols // 256):
        x[b * 256 + (b * 41) % 256] = 127.0
    return w.reshape(-1), x


@pytest.mark.parametrize("qtype,cols,xr", CASES, ids=["Q4_K", "Q6_K", "Q8_0"])
def test_self_check_patterns_are_exact_in_the_reference_order(oracle_lib, qtype, cols, xr):
    w, x = check_inputs(qtype, cols, xr)
    # d = dmin = 1: every dequantised weight is an integer, so the exact
    # answer is an integer dot
    deq = ref.dequant(qtype, w, ROWS, cols).astype(np.int64)
    want = deq @ x.astype(np.int64)
    assert np.abs(want).max() < 2 ** 24
    got = ref.matvec(qtype, w, x, ROWS, cols)
    assert np.array_equal(got, want.astype(np.float32))
    # and x quantises to itself: Q8K scale exactly 1
    q8, sc = ref.q8k_quantize(x)
    assert np.array_equal(q8.astype(np.float32), x) and (sc == 1.0).all()


def test_self_check_q4k_extremes_answer(oracle_lib):
    """All-0xff Q4_K row (d = dmin = 1), x = 127: 28,675,584 per block
    (TestAuditQ4KDotExtremes, q4k_q8_amd64_audit_test.go:18-52)."""
    cols = 1024
    row = np.full(ref.row_bytes(ref.Q4_K, cols), 0xFF, np.uint8)
    for b in range(cols // 256):
        row[b * 144:b * 144 + 4] = [0x00, 0x3C, 0x00, 0x3C]
    x = np.full(cols, 127.0, np.float32)
    got = ref.matvec(ref.Q4_K, row, x, 1, cols)[0]
    assert got == np.float32(28675584.0 * 4) == np.float32(63 * 15 * 127 * 1024 - 32 * 63 * 32 * 127)
