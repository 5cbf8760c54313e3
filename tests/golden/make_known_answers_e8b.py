"""Writes tests/golden/known_answers_e8b.json: hand-derived 2-bit E8 encoder answers.

Each vector case gives an 8-vector v (already divided by its scale, as at
lattice.py:228) and the codes the reference's rule must produce.  The expected
codes were derived by hand from the rule's definition (lattice.py:230-240), not
computed by the oracle; each case's derivation is in its "why" text.  The rule:
  xs = v - 0.5;  f2 = clamp(round_half_even(xs), -2, 1)
  alt = clamp(f2 + 1, -2, 1) if xs >= f2 else clamp(f2 - 1, -2, 1)
  pen = (alt - xs)^2 - (f2 - xs)^2
  if sum(f2) is odd: f2[first argmin pen] = alt[...]
  code = f2 + 2  (w_e8 = f2 + 0.5, code = clamp(round(w_e8 + 1.5), 0, 3))

Group cases have scales that are exact in fp32 (sum of squares and square roots
exact), so the whole pack (scale, codes, bytes c0 | c1<<2 | c2<<4 | c3<<6 at
lattice.py:242-247, fp16 scale) is known in closed form.
"""

import json
import os

cases = [
    dict(v=[0.0] * 8, codes=[2] * 8,
         why="xs = -0.5 -> round half to even = -0 -> f2 = -0, sum 0 even; code = 2 (w_e8 = +0.5)"),
    dict(v=[0.5] * 8, codes=[2] * 8,
         why="xs = 0 -> f2 = 0, even; code 2"),
    dict(v=[1.0] + [0.5] * 7, codes=[2] * 8,
         why="xs0 = 0.5 -> round half to even = 0; others 0; even; all code 2"),
    dict(v=[1.6] + [0.5] * 7, codes=[3] + [2] * 7,
         why="xs0 = 1.1 -> f2 1, sum 1 odd; coord 0: xs >= f2 so alt = clamp(2) = 1 = f2, "
             "pen 0; coords 1..7: xs 0, alt 1, pen 1; argmin 0 -> 'flip' to 1 changes nothing: "
             "the vector keeps its odd sum (clamp quirk)"),
    dict(v=[1.3] + [0.5] * 7, codes=[2] * 8,
         why="xs0 = 0.8 -> f2 1, odd; coord 0: xs < f2 so alt 0, pen 0.64 - 0.04 = 0.6; "
             "others pen 1; argmin 0 -> f2 = 0; all code 2"),
    dict(v=[0.5] * 7 + [1.5], codes=[2] * 7 + [3],
         why="xs7 = 1.0 -> f2 1, odd; coord 7: xs >= f2, alt = clamp(2) = 1, pen 0; "
             "others pen 1; argmin 7, no change (clamp quirk)"),
    dict(v=[1.25, 1.25, 1.25] + [0.5] * 5, codes=[2, 3, 3, 2, 2, 2, 2, 2],
         why="xs 0.75 x3 -> f2 1 x3, sum 3 odd; coords 0..2: alt 0, pen 0.5625 - 0.0625 = 0.5; "
             "others pen 1; first argmin 0 -> f2[0] = 0"),
    dict(v=[-1.0] * 8, codes=[0] * 8,
         why="xs = -1.5 -> round half to even = -2; sum -16 even; code 0 (w_e8 = -1.5)"),
    dict(v=[-3.0] + [0.5] * 7, codes=[0] + [2] * 7,
         why="xs0 = -3.5 -> round -4 -> clamp -2; sum -2 even; code 0"),
    dict(v=[-3.0, 1.6] + [0.5] * 6, codes=[0, 3] + [2] * 6,
         why="f2 = [-2, 1, 0..], sum -1 odd; coord 0: xs -3.5 < f2 so alt = clamp(-3) = -2, "
             "pen 0; coord 1: xs 1.1 >= 1, alt 1, pen 0; argmin 0 (first of the ties), "
             "no change: odd sum kept"),
    dict(v=[0.0, 1.6] + [0.5] * 6, codes=[1, 3] + [2] * 6,
         why="f2 = [-0, 1, 0..], sum 1 odd; coord 0: xs -0.5 < f2 (-0) so alt = -1, "
             "pen 0.25 - 0.25 = 0; coord 1: pen 0; argmin 0 -> f2[0] = -1, code 1; sum 0"),
    dict(v=[2.0] + [0.5] * 7, codes=[3] + [2] * 7,
         why="xs0 = 1.5 -> round half to even = 2 -> clamp 1; sum 1 odd; coord 0 alt "
             "clamp(2) = 1, pen 0; argmin 0, no change"),
    dict(v=[0.25] * 8, codes=[2] * 8,
         why="xs = -0.25 -> round = -0; sum 0 even; code 2"),
    dict(v=[-0.25, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 2.2], codes=[1, 2, 2, 2, 2, 2, 2, 3],
         why="xs0 = -0.75 -> f2 -1; xs7 = 1.7 -> round 2 -> clamp 1; sum 0 even; "
             "codes 1 and 3"),
]

groups = [
    dict(w=[1.0] * 8, gs=8, scale16=0x3C00, codes=[2] * 8,
         why="sum of squares 8, norm sqrt(8) = fp32(sqrt 8) = root, s = 1 (+1e-8 rounds "
             "away); v = 1, xs = 0.5 -> 0; bytes 0xAA 0xAA"),
    dict(w=[2.0] * 8, gs=8, scale16=0x4000, codes=[2] * 8,
         why="norm sqrt(32) = 2 sqrt(8) exactly in fp32, s = 2; v = 1; codes 2"),
    dict(w=[3.0, -3.0] * 4, gs=8, scale16=0x4200, codes=[2, 0] * 4,
         why="norm sqrt(72) = 3 sqrt(8) in fp32, s = 3; v = +-1; xs = 0.5 -> 0, "
             "-1.5 -> -2 (half to even); sum -8 even; codes 2, 0; bytes 0x22 0x22"),
    dict(w=[0.0] * 8, gs=8, scale16=0x0000, codes=[2] * 8,
         why="all zero: norm 0, s = 1e-8 -> fp16 0; v = 0; xs -0.5 -> -0; codes 2"),
]


def byte_of(c):
    return c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6)


for g in groups:
    g["bytes"] = [byte_of(g["codes"][4 * i:4 * i + 4]) for i in range(len(g["codes"]) // 4)]

out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers_e8b.json")
with open(out, "w") as f:
    json.dump(dict(vectors=cases, groups=groups), f, indent=1)
print(out)
