"""The ternary encoder kernel's reduced penalty form (csrc/e8t_codec.hip, quantize8).

TernaryE8LatticePacker.pack (ojasx2/math/lattice.py:357-373) fixes an odd 8-vector by
flipping the coordinate with the first smallest pen = (alt - v)^2 - (q - v)^2, each operation
rounded in fp32, with q = clamp(rint(v), -1, 1) and alt = q == 0 ? (v >= 0 ? 1 : -1) : 0.
The kernel evaluates instead d = fl(1 - |v|), t = fl(fl(d * d) - fl(v * v)) and relies on
  pen == |t|                         for every finite v, and
  alt - q == sgn(v) * sgn(t)         for every v with |v| < 2^24, with sgn(-0) = +1 (the
                                     reference's alt is +1 for v = -0, since -0 >= 0).
The kernel's quotient v can be -0 (a negative subnormal weight over a scale >= 2), so the
kernel takes v's sign from v < 0, not from its sign bit, and this test includes -0.
Both were checked over all 2^32 fp32 bit patterns when the kernel was written; this test
re-checks every fp32 value with |v| < 8 (the kernel's range is |v| <= sqrt(gs)(1 + eps)) at a
stride, densely around the decision points 0.5 and 1.5, and at the extremes.  numpy's float32
arithmetic rounds every operation to nearest-even, as the reference's torch CPU ops do.
"""

import numpy as np


def _check(bits: np.ndarray) -> None:
    bits = bits[(bits & 0x7F800000) != 0x7F800000]   # finite only
    v = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        _check_values(v)


def _check_values(v: np.ndarray) -> None:
    one = np.float32(1.0)
    q = np.clip(np.rint(v), -one, one)
    alt = np.where(q == 0, np.where(v >= 0, one, -one), np.float32(0.0)).astype(np.float32)
    a = alt - v
    b = q - v
    pen = a * a - b * b
    d = one - np.abs(v)
    t = d * d - v * v
    assert pen.dtype == np.float32 and t.dtype == np.float32
    assert np.array_equal(pen, np.abs(t), equal_nan=True), "pen != |t|"  # both NaN past ~1.8e19
    small = np.abs(v) < np.float32(2.0 ** 24)
    sign = (v < 0) ^ ((t.view(np.uint32) & np.uint32(0x80000000)) != 0)
    flip = np.where(sign, -one, one)
    assert np.array_equal((alt - q)[small], flip[small]), "alt - q != sgn(v) sgn(t)"


def test_reduced_form_minus_zero():
    # v = -0: q = 0 and alt = +1 (the reference tests v >= 0); the sign bit of v would say -1
    _check(np.array([0x80000000, 0x00000000], dtype=np.uint32))
    v = np.array([-0.0], dtype=np.float32)
    sign_bit = (v.view(np.uint32) & np.uint32(0x80000000)) != 0
    assert sign_bit[0] and not (v < 0)[0]


def test_reduced_form_strided_below_8():
    top = np.float32(8.0).view(np.uint32)
    for start in range(0, int(top), 1 << 26):
        pos = np.arange(start, min(start + (1 << 26), int(top)), 13, dtype=np.uint32)
        _check(pos)
        _check(pos | np.uint32(0x80000000))


def test_reduced_form_dense_near_decision_points():
    for c in (0.5, 1.0, 1.5, 2.0, 0.25):
        mid = int(np.float32(c).view(np.uint32))
        pos = np.arange(mid - (1 << 20), mid + (1 << 20), dtype=np.uint32)
        _check(pos)
        _check(pos | np.uint32(0x80000000))


def test_reduced_form_tiny_and_huge():
    pos = np.concatenate([np.arange(0, 1 << 20, dtype=np.uint32),                    # subnormals, +0
                          np.arange(0x4B000000, 0x4B000000 + (1 << 16), dtype=np.uint32),  # ~2^23
                          np.arange(0x7F000000, 0x7F800000, 97, dtype=np.uint32)])        # huge
    _check(pos)
    _check(pos | np.uint32(0x80000000))
