"""The finish kernel's l / T for the deep draw's bins: q0 = l r with r = 1/T
rounded, then q0 + (l - q0 T) r in two fused multiply-adds
(div_by_temperature). The kernel's bins and gathered keys rely on it being
l / T correctly rounded, the reference's value (sampling.ts:34). Checked here
without a GPU: each fused multiply-add is evaluated exactly in rational
arithmetic and rounded once, as the hardware does, and compared with the
correctly rounded quotient, over float logits and temperatures in
[2^-20, 2^20]."""
import math
import random
import struct
from fractions import Fraction


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))  # one rounding


def div_by_temperature(l, T, r):
    q0 = l * r
    return fma(fma(-q0, T, l), r, q0)


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def cases(n, seed):
    rng = random.Random(seed)
    temps = [0.7, 0.8, 1.0, 1.5, 0.5, 0.3, 0.6, 0.9, 1.1, 1.3, 2.0, 0.05, 3.7, 0.123456789]
    for i in range(n):
        if i % 2:
            T = math.ldexp(1.0 + rng.getrandbits(52) * 2.0 ** -52, rng.randint(-20, 20))
        else:
            T = temps[i % len(temps)]
        if i % 3 == 0:
            bits = rng.getrandbits(32)
            l = struct.unpack("<f", struct.pack("<I", bits))[0]
            if not math.isfinite(l):
                continue
        else:
            l = f32(rng.uniform(-40.0, 40.0))
        yield l, T


def test_correctly_rounded_quotient():
    n = 0
    for l, T in cases(30000, 11):
        r = 1.0 / T
        assert div_by_temperature(l, T, r) == l / T, (l.hex(), T.hex())
        n += 1
    assert n > 25000


def test_the_correction_step_matters():
    """Without the correction the product alone is off in a good share of
    cases: the check above would catch a dropped step."""
    off = sum(1 for l, T in cases(4000, 12) if l * (1.0 / T) != l / T)
    assert off > 200, off


def test_signed_zero_and_extremes():
    for T in (0.7, 2.0 ** -20, 2.0 ** 20):
        r = 1.0 / T
        assert div_by_temperature(0.0, T, r) == 0.0
        assert div_by_temperature(-0.0, T, r) == 0.0  # +0: the keys treat both zeros alike
        big = struct.unpack("<f", struct.pack("<I", 0x7F7FFFFF))[0]
        tiny = struct.unpack("<f", struct.pack("<I", 0x00000001))[0]
        for l in (big, -big, tiny, -tiny):
            assert div_by_temperature(l, T, r) == l / T
