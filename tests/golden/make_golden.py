"""Writes reference_fixtures.json: the known-answer data held in the
reference's own Go tests for this path, transcribed as plain data (inputs and
expected outputs), plus closed-form expectations derived by hand from the
block formats.  No reference source is executed or copied: the Go toolchain
is absent, and these tables are the tests' literal constants.

Run: python tests/golden/make_golden.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

FIXTURES = {
    # kv_f16_test.go:31-54 TestF32ToF16RoundsToNearestEven: (input, f16 bits)
    "f32_to_f16_rne": [
        [0.0, 0x0000], [1.0, 0x3C00], [-2.0, 0xC000], [65504.0, 0x7BFF], [65520.0, 0x7C00],
        [1e9, 0x7C00], ["-inf", 0xFC00], [5.9604645e-8, 0x0001], [1e-10, 0x0000],
        [1.0009765625, 0x3C01], [1.00048828125, 0x3C00], [1.00146484375, 0x3C02],
    ],
    # quant_q8k_portable_amd64_test.go:75-81: exact ties and near-ties checked
    # bit-for-bit against math.RoundToEven (expected values by IEEE RNE).
    "round_to_even": [
        [0.0, 0.0], [-0.0, -0.0], [0.5, 0.0], [-0.5, -0.0], [1.5, 2.0], [-1.5, -2.0],
        [2.5, 2.0], [-2.5, -2.0], [3.5, 4.0], [-3.5, -4.0], [126.5, 126.0], [-126.5, -126.0],
        [127.0, 127.0], [-127.0, -127.0], [127.4999, 127.0], [-127.4999, -127.0],
        [1.0, 1.0], [-1.0, -1.0], [0.4999999, 0.0], [-0.4999999, -0.0],
    ],
    # attention_fastmath_test.go:17-19 score lists (softcap 0 cases); the
    # expected weights are exp(s - max) in float64, denominators their sum.
    "attention_scores": {
        "ordinary": [-9, -3.5, -0.25, 0, 0.7, 3, 9],
        "longTail": [-80, -40, -20, -5, -1, 0],
    },
    # simd_test.go:132-153 TestDequantRowQ4KUsesScalesAndMins: one block,
    # d = 1 (0x3c00), dmin = 0, scale bytes as below, every nibble byte 0x21
    # -> the low-nibble halves decode to 1, the high-nibble halves to 2.
    "q4k_dequant_known": {
        "header": [0x00, 0x3C, 0x00, 0x00],
        "scales": [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1],
        "qbyte": 0x21,
        "expect_low": 1.0,
        "expect_high": 2.0,
    },
    # q4k_q8_amd64_audit_test.go:18-52 TestAuditQ4KDotExtremes: cols 1024,
    # d = dmin = 1, every scale/quant byte 0xff (sc = m = 63, nibble 15),
    # x = +-1.  Per element d*sc*q - dmin*m = 63*15 - 63 = 882, so the row
    # dot is +-882 * 1024; the exact int32 lane sum per block is
    # 63*15*127*32 = 3,840,480 (x sign).
    "q4k_extremes": {"cols": 1024, "expect": 903168.0, "lane_int": 3840480},
    # q4k_q8_amd64_audit_test.go:55-89 TestAuditQ6KDotExtremes: quants 63,
    # scales +127 / -128, d = 1, x = +-1: per element d*sc*(63-32) = 31*sc.
    "q6k_extremes": {"cols": 1024, "scale_bytes": [0x7F, 0x80],
                     "expect_per_scale": {"127": 31744.0 * 127, "-128": -31744.0 * 128}},
    # q8_0_q8_amd64_test.go:64-98 TestAuditQ8_0DotExtremes: w = +-127,
    # d = 1, x = +-1: per element 127.
    "q8_0_extremes": {"cols": 1024, "expect": 130048.0},
    # Deterministic-pattern inputs (no RNG) of the lane-order audits:
    # q4k_q8_amd64_audit_test.go:93-152 and :189-226.
    "lane_order_q4k": {"cols": 512, "scale_byte": "(i*37 + b*11) & 0xff",
                       "quant_byte": "(i*89 + b*7) & 0xff", "x": "((i % 97) - 48) / 48",
                       "d": 0x3C00, "dmin": 0x3000},
    "lane_order_q6k": {"cols": 512, "byte": "(i*131 + b*17) & 0xff", "x": "((i % 89) - 44) / 44",
                       "d": 0x3C00},
    "q8k_quantize_edges": {"cols": 1024, "x": "((i % 53) - 26) / 26",
                           "zero_ranges": [[256, 768]], "x767": -3.5},
    # kernel_bench.go:205-211 deterministicBenchVector: ((i % 251) - 125) / 125
    "bench_vector": "((i % 251) - 125) / 125",
}


def main():
    path = os.path.join(HERE, "reference_fixtures.json")
    with open(path, "w") as f:
        json.dump(FIXTURES, f, indent=1, sort_keys=True)
    print(path)


if __name__ == "__main__":
    main()
