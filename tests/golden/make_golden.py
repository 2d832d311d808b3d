"""Writes the known-answer fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference ships no golden-vector files, so these are derived here, independently of oracle/:
  quant_known.json   int8 / q4 row quantisation (scripts/quantize_table_eval.py:55-61, smlm/kernels.py:280-300)
                     computed in exact rational arithmetic with explicit IEEE round-to-nearest-even to fp16 and
                     fp32 and round-half-even to integers -- no numpy/torch conversion is used for the answers.
  select_known.json  product-key selection cases (smlm/kernels.py:146-177) whose answer follows from how the
                     case is built (ties everywhere, signed zeros, pruned pairs); the expected indices are
                     enumerated below from that construction.
"""
import json
import math
import os
import struct
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))


# ------------------------------------------------------------------ exact IEEE rounding of rationals
def _round_half_even(x):
    """Fraction -> nearest integer, ties to even."""
    f = math.floor(x)
    r = x - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        return f + 1
    return f


def _round_float(x, mant_bits, min_exp):
    """Round a Fraction to a binary float with `mant_bits` fraction bits and minimum normal exponent `min_exp`
    (round to nearest, ties to even; subnormals below 2**min_exp; no overflow handling needed here)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, min_exp)
    ulp = Fraction(2) ** (e - mant_bits)
    return sign * _round_half_even(a / ulp) * ulp


def fp16(x):
    return _round_float(x, 10, -14)


def fp32(x):
    return _round_float(x, 23, -126)


def f32_literal(v):
    """Exact value of the fp32 nearest to the decimal literal v (the test's input)."""
    return Fraction(struct.unpack("<f", struct.pack("<f", v))[0])


def fp16_bits(x):
    return struct.unpack("<H", struct.pack("<e", float(x)))[0]  # x is exactly representable here


def quantize_row(row, lo, hi):
    vals = [f32_literal(v) for v in row]
    best = 0
    for i, v in enumerate(vals):                # first index of the largest magnitude
        if abs(v) > abs(vals[best]):
            best = i
    d = fp16(vals[best] / lo)
    if d == 0:
        d = Fraction(1)
    codes = [min(max(_round_half_even(fp32(v / d)), lo), hi) for v in vals]
    return codes, d


def quant_fixture():
    rows_i8 = [
        # m = -1.0 -> d = 2^-7; 0.3 -> 38.4 -> 38; 1.5 -> 2 and 2.5 -> 2 (half-even); -3.5 -> -4; 126.72 -> 127
        [0.5, -1.0, 0.25, 0.3, 0.01171875, 0.01953125, -0.02734375, 0.99],
        [0.0] * 8,                                        # d would be 0 -> 1, all codes 0
        [-0.5, 0.5, 0.25, 0.0, 0.125, -0.0625, 0.375, 0.1],   # first of the tied |max| is -0.5; +0.5 -> 128 -> 127
        [0.3, -0.1, 0.2, 0.05, -0.25, 0.15, 0.01, -0.2999],  # positive m: fp16(0.3 / -128) needs rounding
        [1e-3, -7e-4, 3.3e-4, 9.99e-4, -1e-3, 5e-5, 0.0, 2.5e-4],  # tiny scale, fp16 subnormal-adjacent
    ]
    rows_q4 = [
        [1.0, -0.5, 0.25, 0.1875, -0.3125, 0.0625, -1.0, 0.9],  # m = 1.0 (first), d = -0.125
        [0.0] * 8,
        [-0.7, 0.2, 0.35, -0.05, 0.61, -0.69, 0.1, 0.0],
    ]
    out = {"i8": [], "q4": []}
    for row in rows_i8:
        codes, d = quantize_row(row, -128, 127)
        out["i8"].append({"row": row, "codes": codes, "scale_f16_bits": fp16_bits(d)})
    for row in rows_q4:
        codes, d = quantize_row(row, -8, 7)
        half = len(row) // 2
        packed = [(codes[i] + 8) | ((codes[half + i] + 8) << 4) for i in range(half)]
        out["q4"].append({"row": row, "codes": codes, "packed": packed, "scale_f16_bits": fp16_bits(d)})
    return out


# ------------------------------------------------------------------ selection cases
BF16_ONE, BF16_PZERO, BF16_NZERO = 0x3F80, 0x0000, 0x8000


def pruned_pairs(knn):
    return [(i, j) for i in range(knn) for j in range(knn) if (i + 1) * (j + 1) <= knn]


def select_fixture():
    cases = []
    NK, knn = 64, 8
    # 1. every score equal: both halves rank sub-keys 0, 1, 2, ... (ties -> lower index); every candidate ties,
    #    so the knn lowest table indices i1*NK + i2 among the pruned pairs win: pairs (0, j) give 0..knn-1.
    cases.append({"name": "all_equal", "NK": NK, "knn": knn, "s1": [BF16_ONE] * NK, "s2": [BF16_ONE] * NK,
                  "idx": list(range(knn)), "score_bits": [0x4000] * knn})
    # 2. signed zeros: in s1 only sub-key 5 is +0, all others -0, so +0 ranks first: ranks -> sub-keys
    #    5, 0, 1, 2, 3, 4, 6, 7; s2 is all +0 (ranks -> 0..7).  Every candidate sum is +0 (-0 + +0 = +0), so the
    #    winners are the knn lowest i1[i]*NK + i2[j] over pairs with (i+1)(j+1) <= knn.  Pairs beyond that
    #    (e.g. rank 1 x rank 4 = sub-keys (0, 4) -> index 4) are pruned, so index 4 is NOT selected.
    s1 = [BF16_NZERO] * NK
    s1[5] = BF16_PZERO
    ranks1 = [5, 0, 1, 2, 3, 4, 6, 7]
    ranks2 = list(range(knn))
    cand = sorted(ranks1[i] * NK + ranks2[j] for i, j in pruned_pairs(knn))
    cases.append({"name": "signed_zero_pruned", "NK": NK, "knn": knn, "s1": s1, "s2": [BF16_PZERO] * NK,
                  "idx": cand[:knn], "score_bits": [BF16_PZERO] * knn})
    # 3. distinct powers of two: s1[k] = 2^-(k+1), s2[k] = 2^-(k+1) for k < 16, zero (+0) elsewhere.  The
    #    candidate (i, j) scores 2^-(i+1) + 2^-(j+1), exact in fp32 and in bf16 when |i - j| <= 7.  Order by
    #    score: (0,0)=1, then (0,1),(1,0)=0.75, (0,2),(2,0)=0.625, (1,1)=0.5 ... the top 8 with ties -> lower
    #    index: (0,0), (0,1)=1, (1,0)=64, (0,2)=2, (2,0)=128, (0,3)=3, (3,0)=192, then 0.5: (1,1)=65 ties with
    #    (0,4)=0.53125? no: 2^-1 + 2^-5 = 0.53125 > 0.5, so (0,4)=4 is 8th.
    s = [BF16_PZERO] * NK
    for k in range(16):
        s[k] = (127 - (k + 1)) << 7            # bf16 bits of 2^-(k+1)
    # scores 1, 0.75, 0.75, 0.625, 0.625, 0.5625, 0.5625, 0.53125 as bf16 bit patterns
    cases.append({"name": "powers_of_two", "NK": NK, "knn": knn, "s1": s, "s2": s,
                  "idx": [0, 1, 64, 2, 128, 3, 192, 4],
                  "score_bits": [0x3F80, 0x3F40, 0x3F40, 0x3F20, 0x3F20, 0x3F10, 0x3F10, 0x3F08]})
    return {"cases": cases}


def main():
    with open(os.path.join(HERE, "quant_known.json"), "w") as f:
        json.dump(quant_fixture(), f, indent=1)
    with open(os.path.join(HERE, "select_known.json"), "w") as f:
        json.dump(select_fixture(), f, indent=1)
    print("wrote quant_known.json, select_known.json")


if __name__ == "__main__":
    main()
