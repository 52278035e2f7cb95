#!/usr/bin/env python3
"""Write tests/golden/q8_vectors.json: Q8 activation cases whose answers are
fixed by construction, not by running any quantizer.

The reference quantizer (src/quant.rs:904-922, :965-991) is
    max = max|x| over a 256-group; (s, inv) = (max/127, 127/max) or (0, 0);
    q = saturate_i8(round_half_even(x * inv)) for 16-element steps,
    q = clamp(round_half_away(x * inv), -127, 127) for a group's tail.
Every finite case below has max|x| = 127 in each group, so inv = 127/127 =
1.0 and s = 1.0 exactly, which makes q = round(x) with the stated tie rule.
Values are halves and quarters (exact in f32), so the expected integers
follow from Python's own integer arithmetic.

Non-finite values follow the aarch64 instructions the reference uses:
max_abs_neon (src/quant.rs:869-892) takes vmaxq_f32 / vmaxvq_f32 (FMAX,
FMAXV: NaN if either operand is NaN) over the 16-value steps, then folds the
tail with f32::max (a NaN operand yields the other). A NaN maximum fails
`max > 0.`, so (s, inv) = (0, 0) and every code is 0 (x * 0 is 0 or NaN, and
vcvtnq_s32_f32 / `as i8` turn NaN into 0). An infinite maximum gives s = inf,
inv = 0, so again every code is 0. Since JSON has no NaN or infinity, every
case also carries its inputs and scales as f32 bit patterns (x_bits,
scales_bits), which the tests read.
"""
import json
import math
import os
import struct
from fractions import Fraction

NAN = float("nan")
INF = float("inf")


def f32_bits(v: float) -> str:
    return "%08x" % struct.unpack("<I", struct.pack("<f", v))[0]


def half_even(v: Fraction) -> int:
    return round(v)  # Python rounds Fractions half to even


def half_away(v: Fraction) -> int:
    f = abs(v)
    n = int(f)
    if f - n >= Fraction(1, 2):
        n += 1
    return n if v >= 0 else -n


def group_max(grp):
    """max_abs_neon: NaN-propagating over the 16-value steps, then the tail
    folded by f32::max (a NaN operand yields the other)."""
    vec = len(grp) // 16 * 16
    body = [abs(v) for v in grp[:vec]]
    mx = NAN if any(math.isnan(v) for v in body) else max(body, default=0.0)
    for v in grp[vec:]:
        a = abs(v)
        if math.isnan(mx):
            mx = a
        elif not math.isnan(a):
            mx = max(mx, a)
    return mx


def case(name, values):
    q, scales = [], []
    for g0 in range(0, len(values), 256):
        grp = values[g0:g0 + 256]
        mx = group_max(grp)
        if not mx > 0 or math.isinf(mx):
            # (0, 0) for a zero or NaN maximum, (inf, 0) for an infinite one:
            # every product x * inv is 0 or NaN, and NaN converts to 0
            scales.append(INF if math.isinf(mx) else 0.0)
            q.extend([0] * len(grp))
            continue
        assert mx == 127, name
        scales.append(1.0)
        vec = len(grp) // 16 * 16
        for i, v in enumerate(grp):
            if math.isnan(v):
                q.append(0)
                continue
            v = Fraction(v)
            r = half_even(v) if i < vec else max(-127, min(127, half_away(v)))
            q.append(max(-128, min(127, r)))
    shown = [v if math.isfinite(v) else str(v) for v in values]
    return {"name": name, "x": shown, "x_bits": [f32_bits(v) for v in values], "q": q,
            "scales": [v if math.isfinite(v) else str(v) for v in scales],
            "scales_bits": [f32_bits(v) for v in scales]}


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
    # a NaN in a group's 16-value steps: that group's scale and codes are 0,
    # the next group is quantized as usual
    nan_body = list(live)
    nan_body[37] = NAN
    cases.append(case("nan_in_body", nan_body + live))
    # a NaN in the tail of a partial group is skipped by the maximum and
    # converts to code 0
    cases.append(case("nan_in_tail", live + live[:16] + [2.5, NAN, -126.5, 127.0]))
    # a NaN in the steps of a partial group whose tail holds the maximum: the
    # tail's value replaces the NaN maximum, and body values above it
    # saturate (vqmovn: 200 -> 127, -300 -> -128)
    body16 = [1.5, NAN, 200.0, -300.0] + [float(k) for k in range(-6, 6)]
    cases.append(case("nan_in_body_with_tail", live + body16 + [127.0, -0.5, 0.5, 3.0]))
    # an infinite value: scale inf, inverse 0, every code of the group 0
    inf_grp = list(live)
    inf_grp[200] = -INF
    cases.append(case("infinity", live + inf_grp))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q8_vectors.json")
    with open(out, "w") as f:
        json.dump(cases, f, indent=1)
        f.write("\n")
    print("wrote", out)


if __name__ == "__main__":
    main()
