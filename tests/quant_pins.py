"""Known-answer quantizer blocks that fix the reference's rounding order.

The reference quantizes with id = 1.0f/d and a separate f32 product x*id
(kv.h:406-410), then for the nibble types a separate f32 add of the offset
before the truncation (kv.h:428-432,459-463,491-495). Each block below holds
elements where that order gives a different code than the two plausible
alternatives: dividing by d directly (x/d), or a fused multiply-add of the
offset (one rounding of x*id + c). The expected codes are derived here by
exact rational arithmetic with IEEE binary32 round-to-nearest-even at every
step the reference rounds (independent of the oracle's C code), and each block
asserts that at least one alternative order changes a code.
"""
import math
from fractions import Fraction as F

import numpy as np


def f32(r):
    """The binary32 value nearest to the rational r (ties to even), normal range."""
    r = F(r)
    if r == 0:
        return F(0)
    s = -1 if r < 0 else 1
    a = abs(r)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while F(2) ** e > a:
        e -= 1
    while F(2) ** (e + 1) <= a:
        e += 1
    ulp = F(2) ** (e - 23)
    m = a / ulp
    n = math.floor(m)
    fr = m - n
    if fr > F(1, 2) or (fr == F(1, 2) and n % 2 == 1):
        n += 1
    return s * n * ulp


def roundf(v):
    """C roundf: half away from zero."""
    return int(math.floor(abs(v) + F(1, 2))) * (1 if v >= 0 else -1)


def trunc(v):
    return int(v) if v >= 0 else -int(-v)


def block(vals):
    x = np.zeros(32, np.float32)
    x[: len(vals)] = np.float32(vals)
    return x


# (values; the first one(s) set the block's scale)
Q8_0_BLOCK = [1.6334146, -0.23793833, -0.77812266, 0.81670725, 1.2282763]
Q4_0_BLOCK = [1.9903495, -1.1195714, 0.12439691, -0.8707778]
Q5_0_BLOCK = [-2.0363986, -0.19091244, 0.8272868, 1.7182112, 0.19091225]
Q4_1_BLOCK = [-1.8538204, 2.3112106, -1.7149861, 1.0617012, -0.048973713, 0.22869514]


def q8_0_codes(x):
    """kv.h:402-411: d = amax/127, id = 1/d, q = roundf(x*id); returns (codes,
    codes by roundf(x/d))."""
    xs = [F(float(v)) for v in x]
    amax = max(abs(v) for v in xs)
    d = f32(amax / 127)
    idv = f32(1 / d) if d else F(0)
    ref = [roundf(f32(v * idv)) for v in xs]
    div = [roundf(f32(v / d)) if d else 0 for v in xs]
    return ref, div


def signed_absmax(xs):
    amax, vmax = F(0), F(0)
    for v in xs:
        if amax < abs(v):
            amax, vmax = abs(v), v
    return vmax


def nib_codes(kind, x):
    """q4_0 (kv.h:476-499), q5_0 (kv.h:412-445), q4_1 (kv.h:446-467): returns
    (codes in the reference order, codes with a fused offset add, codes by x/d),
    each clamped as the reference clamps."""
    xs = [F(float(v)) for v in x]
    if kind == "q4_1":
        lo, hi = min(xs), max(xs)
        d = f32((hi - lo) / 15)
        xs = [f32(v - lo) for v in xs]
        c, top = F(1, 2), 15
    else:
        div_c, c, top = (8, F(17, 2), 15) if kind == "q4_0" else (16, F(33, 2), 31)
        d = f32(signed_absmax(xs) / -div_c)
    idv = f32(1 / d)
    clamp = lambda q: min(max(q, 0), top)
    ref = [clamp(trunc(f32(f32(v * idv) + c))) for v in xs]
    fused = [clamp(trunc(f32(v * idv + c))) for v in xs]
    div = [clamp(trunc(f32(f32(v / d) + c))) for v in xs]
    return ref, fused, div


def decode_codes(kind, raw):
    """Element codes of one stored block (bytes in the reference's layout)."""
    raw = np.asarray(raw, np.uint8)
    if kind == "q8_0":
        return list(raw[2:34].view(np.int8).astype(int))
    if kind == "q4_0":
        qs = raw[2:18]
        return list(np.concatenate([qs & 15, qs >> 4]).astype(int))
    if kind == "q4_1":
        qs = raw[4:20]
        return list(np.concatenate([qs & 15, qs >> 4]).astype(int))
    qh = int(raw[2]) | int(raw[3]) << 8 | int(raw[4]) << 16 | int(raw[5]) << 24
    qs = raw[6:22]
    low = np.concatenate([qs & 15, qs >> 4]).astype(int)
    return [int(low[e]) | ((qh >> e) & 1) << 4 for e in range(32)]
