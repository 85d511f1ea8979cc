"""The deep draw's arithmetic, pinned without a GPU (gs_finish.hip): the
quartic table exponential exp2_256_tight (last-bin terms and bin scales) and
the bin-centred units of deep_units. Every binary64 step is evaluated in
exact rationals and rounded once, as the kernel's fma / multiply do, and
compared with high-precision exponentials."""
import os
import re
from decimal import Decimal, getcontext
from fractions import Fraction

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "gemma-webgpu-engine_amd", "csrc", "gs_exp2_table.h")
BINS, SPAN = 4096, 40.0
W = SPAN / BINS


def constants():
    text = open(HEADER).read()
    table_text = text[text.index("GS_EXP2_TABLE_256"):text.index("// Taylor")]
    table = [float.fromhex(h) for h in re.findall(r"0x[0-9a-f.]+p[-+]\d+", table_text)]
    consts = {k: float.fromhex(v) for k, v in re.findall(r"#define (GS_\w+) (0x[0-9a-f.]+p[-+]\d+)", text)}
    return table, consts


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def mul(a, b):
    return float(Fraction(a) * Fraction(b))


def exp2_256_tight(y, table, c):
    n = round(y)
    s = y - n
    p = fma(s, c["GS_EXP2_256_C4"], c["GS_EXP2_256_C3"])
    p = fma(s, p, c["GS_EXP2_256_C2"])
    p = fma(s, p, c["GS_EXP2_256_C1"])
    p = fma(s, p, 1.0)
    return mul(table[n & 255], p) * 2.0 ** (n >> 8)


def deep_units(z, b, c4=1.0 / 24.0):
    x = fma(-z, W, fma(float(b), W, 0.5 * W))
    p = fma(x, c4, 1.0 / 6.0)
    p = fma(x, p, 0.5)
    p = fma(x, p, 1.0)
    p = fma(x, p, 1.0)
    q = fma(p, 2.0 ** 40, 2.0 ** 52)
    return int(q) - 2 ** 52


def test_quartic_constants():
    getcontext().prec = 40
    _, c = constants()
    r = Decimal(2).ln() / 256
    assert c["GS_EXP2_256_C3"] == float(r ** 3 / 6)
    assert c["GS_EXP2_256_C4"] == float(r ** 4 / 24)


def test_exp2_256_tight_relative_error():
    getcontext().prec = 40
    table, c = constants()
    worst = 0.0
    for n in (-22160, -5000, -300, -1, 0, 255, -257):
        for k in range(-50, 51):
            y = n + k / 100.0
            got = exp2_256_tight(y, table, c)
            exact = (Decimal(y) / 256 * Decimal(2).ln()).exp()
            worst = max(worst, float(abs((Decimal(got) - exact) / exact)))
    assert worst < 1e-15, worst


def test_bin_units_relative_error():
    """deep_units(z, b) 2^-40 against e^((b + 1/2 - z) w), over z across
    bins: within 5e-13 relative (the units' rounding, 4.6e-13, dominates)."""
    getcontext().prec = 40
    worst = 0.0
    for b in (0, 1, 7, 100, 2047, 4094):
        for k in range(0, 101):
            z = b + k / 100.0 * (1 - 2.0 ** -30)
            got = Decimal(deep_units(z, b)) / Decimal(2 ** 40)
            x = (Decimal(b) + Decimal("0.5") - Decimal(z)) * Decimal(W)
            exact = x.exp()
            worst = max(worst, float(abs((got - exact) / exact)))
    assert worst < 5e-13, worst


def test_bin_units_catch_a_wrong_coefficient():
    """A mistyped Taylor coefficient (1/12 for 1/24) shows as a larger
    error than the bound above allows, so the check pins the polynomial."""
    getcontext().prec = 40
    worst = 0.0
    for k in range(0, 101):
        z = 5 + k / 100.0
        got = Decimal(deep_units(z, 5, c4=1.0 / 12.0)) / Decimal(2 ** 40)
        exact = ((Decimal(5.5) - Decimal(z)) * Decimal(W)).exp()
        worst = max(worst, float(abs((got - exact) / exact)))
    assert worst > 5e-13, worst


def test_bin_units_fit_u64():
    """A bin holds at most 2^21 + 2048 terms; each is under 2^40 e^(w/2)
    units, so the sum stays below 2^63."""
    top = deep_units(0.0, 0)  # the largest term of a bin: x = w/2
    assert top < 2 ** 40 * 1.005
    assert top * (2 ** 21 + 2048) < 2 ** 63
