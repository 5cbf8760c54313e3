"""Writes tests/golden/known_answers.json: hand-derived encoder answers.

Each case gives an 8-vector v (already divided by its scale, as at
lattice.py:357) and the code the reference's rule must produce.  The expected
codes were derived by hand from the rule's definition, not computed by the
oracle; the derivation of each case is in its "why" text.  The rule
(lattice.py:359-373): q = clamp(round_half_even(v), -1, 1); if sum(q) is odd,
flip the first index of the minimum of pen = (alt - v)^2 - (q - v)^2 to
alt = (q == 0 ? (v >= 0 ? +1 : -1) : 0); code = sum((q_i + 1) 3^i) / 2.

Also holds group-level cases where every fp32 step is exact, so the scale is
known in closed form.
"""

import json
import os

POW3 = [1, 3, 9, 27, 81, 243, 729, 2187]


def code_of(q):
    raw = sum((qi + 1) * p for qi, p in zip(q, POW3))
    assert raw % 2 == 0
    return raw // 2


cases = [
    dict(v=[0.0] * 8, q=[0] * 8,
         why="all zero: q = 0, even parity; raw = sum 3^i = 3280"),
    dict(v=[0.5, 0, 0, 0, 0, 0, 0, 0], q=[0] * 8,
         why="round(0.5) = 0 (half to even); parity even, no flip"),
    dict(v=[-0.5, 0.5, 0, 0, 0, 0, 0, 0], q=[0] * 8,
         why="round(+-0.5) = +-0; even"),
    dict(v=[1.5, 0.25, 0, 0, 0, 0, 0, 0], q=[1, 1, 0, 0, 0, 0, 0, 0],
         why="round(1.5) = 2 -> clamp 1; sum 1 odd; pen0 = 1.5^2-0.5^2 = 2, "
             "pen1 = 0.75^2-0.25^2 = 0.5, pen2..7 = 1; argmin = 1 -> q1 = +1"),
    dict(v=[2.5, -2.5, 0, 0, 0, 0, 0, 0], q=[1, -1, 0, 0, 0, 0, 0, 0],
         why="round(+-2.5) = +-2 -> clamp +-1; sum 0 even"),
    dict(v=[0, 0, 0, 0, 0, 0, 0, 1.0], q=[1, 0, 0, 0, 0, 0, 0, 1],
         why="sum 1 odd; every pen = 1 (v=0 -> alt +1: 1-0; v=1 -> alt 0: 1-0); "
             "ties break to the first index 0, v0 >= 0 -> +1"),
    dict(v=["-0.0", 0, 0, 0, 0, 0, 0, 1.0], q=[1, 0, 0, 0, 0, 0, 0, 1],
         why="-0.0 >= 0 is true so alt0 = +1; all pens tie at 1 -> index 0"),
    dict(v=[-0.25, 0, 0, 0, 0, 0, 0, 1.0], q=[-1, 0, 0, 0, 0, 0, 0, 1],
         why="pen0 = 0.75^2 - 0.25^2 = 0.5 < 1 -> flip 0 towards v0 < 0 -> -1"),
    dict(v=[0.75, 0.75, 0.75, 0, 0, 0, 0, 0], q=[0, 1, 1, 0, 0, 0, 0, 0],
         why="q = (1,1,1,0,..) sum 3 odd; pen0..2 = 0.75^2-0.25^2 = 0.5 (alt 0), "
             "pen3..7 = 1; first argmin 0 -> q0 = alt0 = 0"),
    dict(v=[-1.25, 0.375, 0, 0, 0, 0, 0, 0], q=[-1, 1, 0, 0, 0, 0, 0, 0],
         why="q = (-1, 0, ...) odd; pen0 = 1.25^2-0.25^2 = 1.5; pen1 = 0.625^2 - "
             "0.375^2 = 0.25; pen2..7 = 1 -> flip 1 to +1"),
    dict(v=[0.6] * 8, q=[1] * 8,
         why="round(0.6) = 1 everywhere; sum 8 even; no flip"),
]

for c in cases:
    c["code"] = code_of(c["q"])

# Group-level: gs = 32, all 32 weights equal to a = 2^-3.
#   norm: 8 fma lanes each 4 * 2^-6 = 2^-4 (exact), lane sum 2^-1, sqrt(2^-1) is not
#   exact -- so use a = 2^-3 with 32 values: sum of squares = 32 * 2^-6 = 2^-1;
#   sqrt_rn(0.5) = fp32(0.70710678...) = 0x3F3504F3 = fp32(sqrt 32) / 8 exactly
#   (sqrt(0.5) = sqrt(32)/8 and scaling by 2^-3 commutes with rounding);
#   norm / fp32(sqrt 32) = 2^-3 exactly; + fp32(1e-8): ulp(2^-3) = 2^-26 = 1.49e-8,
#   1e-8 > half ulp -> s = 2^-3 + 2^-26.  v = 2^-3 / s = 1 / (1 + 2^-23) -> RN =
#   1 - 2^-23 (0x3F7FFFFE), round -> 1, q = all 1, even -> code 3280 for all 4 codes.
#   scale fp16 = RN16(2^-3 + 2^-26) = 2^-3 = 0x3000.
groups = [
    dict(gs=32, w=[0.125] * 32, codes=[3280] * 4, scale_f16=0x3000,
         scale_f32_hex="0x3e000001",
         why="a = 2^-3 everywhere: s = 2^-3 + 2^-26, v = 1 - 2^-23 -> all +1"),
    dict(gs=32, w=[0.0] * 32, codes=[1640] * 4, scale_f16=0x0000,
         scale_f32_hex="0x322bcc77",
         why="zero group: s = fp32(1e-8) -> fp16 0; v = 0 -> code 1640"),
]

out = dict(quantize8=cases, groups=groups)
path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
with open(path, "w") as f:
    json.dump(out, f, indent=1)
print("wrote", path, len(cases), "vector cases,", len(groups), "group cases")
