"""The device helper div_by_recip (miq_common.h) replaces x / s in FP8 activation
quantization by RN(q + RN(x - q s) r) with r = RN(1 / s), q = RN(x r). This checks, in
exact rational arithmetic, that the construction gives the correctly rounded fp32 quotient
on the inputs the quantizers see: bf16 x with |x| <= amax and s = RN(max(amax, 1e-12) / 448),
and that copying the sign of x back keeps the sign of a zero quotient (-0 / s is -0, which
e4m3 encodes as 0x80, while the last add alone gives +0)."""
from fractions import Fraction

import numpy as np

f32 = np.float32


def _rn32(v: Fraction) -> np.float32:
    """Round a rational to the nearest fp32 (ties to even)."""
    c = f32(float(v))
    best = None
    for cand in (np.nextafter(c, f32(-np.inf)), c, np.nextafter(c, f32(np.inf))):
        key = (abs(Fraction(float(cand)) - v), int(np.array(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return f32(best[1])


def _bf16(v) -> np.float32:
    return np.array(f32(v)).view(np.uint32).__and__(np.uint32(0xFFFF0000)).view(np.float32)[()]


def _div_by_recip(x, s):
    """The device sequence: r = RN(1/s), q = RN(x r), e = RN(x - q s) (fused),
    RN(e r + q) (fused), then the sign of x copied onto the result."""
    r = f32(f32(1) / s)
    q = f32(x * r)
    e = _rn32(Fraction(float(x)) - Fraction(float(q)) * Fraction(float(s)))
    t = _rn32(Fraction(float(e)) * Fraction(float(r)) + Fraction(float(q)))
    if t == 0:  # an exact zero sum is +0 in round-to-nearest
        t = f32(0.0)
    return np.copysign(t, x)


def test_div_by_recip_is_correctly_rounded():
    rng = np.random.default_rng(7)
    for _ in range(4000):
        amax = _bf16(abs(rng.standard_normal()) * 10 ** rng.uniform(-8, 4))
        s = f32(max(amax, f32(1e-12)) / f32(448))
        x = _bf16(amax * f32(rng.uniform(-1, 1)))
        got = _div_by_recip(x, s)
        assert got == f32(x / s), (x, s, got, f32(x / s))


def test_div_by_recip_keeps_the_sign_of_zero():
    for s in (f32(1.0), f32(3.0 / 448), f32(1e-12 / 448)):
        for x in (f32(0.0), f32(-0.0)):
            got = _div_by_recip(x, s)
            assert got == 0 and np.signbit(got) == np.signbit(x / s) == np.signbit(x)
