#!/usr/bin/env python3
"""Write tests/golden/q8_vectors.json: Q8 activation cases whose answers are
fixed by construction, not by running any quantizer.

The reference quantizer (src/quant.rs:904-922, :965-991) is
    max = max|x| over a 256-group; (s, inv) = (max/127, 127/max) or (0, 0);
    q = saturate_i8(round_half_even(x * inv)) for 16-element steps,
    q = clamp(round_half_away(x * inv), -127, 127) for a group's tail.
Every case below has max|x| = 127 in each group, so inv = 127/127 = 1.0 and
s = 1.0 exactly, which makes q = round(x) with the stated tie rule. Values are
halves and quarters (exact in f32), so the expected integers follow from
Python's own integer arithmetic.
"""
import json
import os
from fractions import Fraction


def half_even(v: Fraction) -> int:
    return round(v)  # Python rounds Fractions half to even


def half_away(v: Fraction) -> int:
    f = abs(v)
    n = int(f)
    if f - n >= Fraction(1, 2):
        n += 1
    return n if v >= 0 else -n


def case(name, values):
    xs = [Fraction(v) for v in values]
    q, scales = [], []
    for g0 in range(0, len(xs), 256):
        grp = xs[g0:g0 + 256]
        mx = max(abs(v) for v in grp)
        if mx == 0:
            scales.append(0.0)
            q.extend([0] * len(grp))
            continue
        assert mx == 127, name
        scales.append(1.0)
        vec = len(grp) // 16 * 16
        for i, v in enumerate(grp):
            r = half_even(v) if i < vec else max(-127, min(127, half_away(v)))
            q.append(max(-128, min(127, r)))
    return {"name": name, "x": [float(v) for v in xs], "q": q, "scales": scales}


def main():
    cases = []
    # ties to even in the 16-wide body: 0.5->0, 1.5->2, 2.5->2, -2.5->-2 ...
    body = [127.0] + [k + 0.5 for k in range(-20, 20)] + [-126.5, 126.5, 0.25, -0.75]
    body += [float(i % 7) - 3.0 for i in range(256 - len(body))]
    cases.append(case("ties_to_even", body))
    # +-max -> +-127, and zeros stay zero
    pm = [127.0, -127.0] + [0.0] * 254
    cases.append(case("plus_minus_max", pm))
    # an all-zero group between two live groups: scale 0, q 0 (no division)
    live = [127.0] + [float((i * 37) % 255 - 127) for i in range(1, 256)]
    cases.append(case("zero_group", live + [0.0] * 256 + live))
    # partial last group of 8 values (< 16): tail rounding is half away from zero
    tail = [127.0, 2.5, -2.5, 0.5, -0.5, 3.5, 1.25, -126.5]
    cases.append(case("partial_tail_half_away", live + tail))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q8_vectors.json")
    with open(out, "w") as f:
        json.dump(cases, f, indent=1)
        f.write("\n")
    print("wrote", out)


if __name__ == "__main__":
    main()
