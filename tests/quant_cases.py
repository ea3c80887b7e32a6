"""Test inputs for the q4_0 code rounding: blocks whose codes depend on how x * (1/d) + 8.5 is rounded.

The reference's device quantizer writes q = trunc(x * id + 8.5) (src/kernels/cuda/kv_q4.cu:84), which its compilers
contract into one fused multiply-add (nvcc's default --fmad=true; clang's HIP default contracts too): the product is
not rounded before the sum.  Its host checker rounds the two separately (src/kernels/kv_q4_parity.cpp:79-82).  The two
differ when the product lands within a rounding step of a half-integer boundary.  These blocks put values exactly
there, found with exact rational arithmetic (Python's Fraction), so that which form a quantizer uses shows in its
codes.
"""
from fractions import Fraction

import numpy as np

F32 = np.float32


def f32_rne(q: Fraction) -> np.float32:
    """An exact rational rounded to the nearest binary32, ties to even (finite results only)."""
    if q == 0:
        return F32(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()   # 2^e <= a < 2^(e+2)
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                                             # below the normal range the step is 2^-149
    scaled = a * Fraction(2) ** (23 - e)                         # the significand in units of the last place
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return F32(sign * m * 2.0 ** (e - 23))


def fused_code(x: np.float32, idv: np.float32) -> int:
    s = f32_rne(Fraction(float(x)) * Fraction(float(idv)) + Fraction(17, 2))
    return int(min(15, max(0, int(np.trunc(s)))))


def separate_code(x: np.float32, idv: np.float32) -> int:
    p = f32_rne(Fraction(float(x)) * Fraction(float(idv)))
    s = f32_rne(Fraction(float(p)) + Fraction(17, 2))
    return int(min(15, max(0, int(np.trunc(s)))))


def boundary_blocks(n_blocks: int, seed: int = 4) -> np.ndarray:
    """[n_blocks][32] f32 blocks: value 0 is the block's maximum m (so d = m / -8 and id = 1/d), the other values sit
    where RN(x * id + 8.5) and RN(RN(x * id) + 8.5) truncate to different codes (as many as the search finds), the
    rest are small ordinary values."""
    rng = np.random.default_rng(seed)
    out = np.zeros((n_blocks, 32), F32)
    for b in range(n_blocks):
        while True:
            m = F32(rng.uniform(1.0, 4.0)) * F32(-1 if b % 2 else 1)
            d = F32(m / F32(-8))
            idv = F32(F32(1) / d)
            found = []
            for n in range(1, 16):            # code boundaries: x * id + 8.5 == n
                centre = F32(Fraction(2 * n - 17, 2) / Fraction(float(idv)))
                cand = centre
                for _ in range(40):           # walk a few ulps each way from the boundary
                    for x in (cand, F32(-cand)):
                        if abs(x) < abs(m) and fused_code(x, idv) != separate_code(x, idv):
                            found.append(x)
                    cand = np.nextafter(cand, F32(np.inf) if cand > 0 else F32(-np.inf))
                if len(found) >= 8:
                    break
            if found:
                break
        row = (rng.standard_normal(32).astype(F32) * F32(0.1) * abs(m)).astype(F32)
        row[0] = m
        k = min(len(found), 31)
        row[1:1 + k] = np.array(found[:k], F32)
        out[b] = row
    return out
