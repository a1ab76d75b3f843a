"""Writes known_answers.json: quantization cases whose codes and scales are derived here with exact
rational arithmetic (fractions), independently of the oracle's C code.

Rule being pinned (hy_nomas/kernels.py:33-36, ops.py:41-52): scale = absmax / 127 rounded to fp32 (1 for
an all-zero group); q = x / scale rounded to fp32, then rounded half away from zero (or half to even),
clamped to +-127.  The inputs are chosen so the fp32 quotient is exact (scale a power of two, or a scale
whose quotients are exact), so exact rational rounding of x / scale is the answer.

    python tests/golden/make_known_answers.py
"""
import json
import os
from fractions import Fraction

import numpy as np


def round_half_away(v):
    mag = abs(v) + Fraction(1, 2)
    r = mag.numerator // mag.denominator
    return int(r) * (1 if v >= 0 else -1)


def round_half_even(v):
    f = v.numerator // v.denominator
    rem = v - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2 == 1):
        return int(f) + 1
    return int(f)


def case(name, x, group, rounding="half_away"):
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[1]
    codes, scales = [], []
    for row in x:
        for g0 in range(0, k, group):
            seg = [Fraction(float(v)) for v in row[g0:g0 + group]]
            peak = max(abs(v) for v in seg)
            scale = float(np.float32(float(peak)) / np.float32(127)) if peak > 0 else 1.0
            scales.append(scale)
            s = Fraction(scale)
            for v in seg:
                y = Fraction(float(np.float32(float(v / s))))     # the fp32 quotient
                r = round_half_away(y) if rounding == "half_away" else round_half_even(y)
                codes.append(max(-127, min(127, r)))
    return {"name": name, "shape": list(x.shape), "x": x.ravel().tolist(), "group": group, "kind": "int8",
            "rounding": rounding, "codes": codes, "scales": scales}


def main():
    cases = []
    # peak 127 -> scale 1: ties at k + 0.5 on both sides of zero
    row = np.zeros(128, dtype=np.float32)
    row[0] = 127.0
    row[1:21] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 62.5, -62.5, 126.5, -126.5,
                 0.25, -0.75, 3.0, -3.0, 100.5, -100.5, 0.0, 1.0, -1.0, 64.5]
    cases.append(case("ties_scale_one_away", [row], 128))
    cases.append(case("ties_scale_one_even", [row], 128, "half_even"))
    # peak 254 -> scale 2 (exact): quotients are x / 2
    row2 = np.zeros(128, dtype=np.float32)
    row2[5] = -254.0
    row2[6:14] = [1.0, -1.0, 3.0, -3.0, 5.0, 9.0, 253.0, -2.0]
    cases.append(case("scale_two", [row2], 128))
    # two groups with different peaks and an all-zero group; per-token over the whole row
    row3 = np.zeros(384, dtype=np.float32)
    row3[:4] = [127.0, 63.5, -31.75, 0.5]
    row3[128:132] = [-0.5, 0.25, 0.125, 0.0625]           # peak 0.5 -> scale fp32(0.5 / 127)
    cases.append(case("three_groups", [row3], 128))
    cases.append(case("per_token_row", [row3], 384))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(out, "w") as f:
        json.dump({"quantize": cases}, f, indent=1)
    print(out)


if __name__ == "__main__":
    main()
