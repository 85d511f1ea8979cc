"""The chunk scan's normaliser exponential, pinned without a GPU.

The scan sums e^((l - lmax)/T) as 2^(y/256) with y = 256 log2(e) (l - lmax)/T,
evaluated as table[n & 255] * p(s) * 2^(n >> 8), n = rint(y), s = y - n,
p(s) = 1 + s (C1 + s C2). These tests check the committed constants against
an independent high-precision evaluation, and the evaluation's relative error
against its stated bound (4.2e-10), in exact rational arithmetic that rounds
each binary64 step the way the kernel's fma / multiply do."""
import os
import re
import sys
from decimal import Decimal, getcontext
from fractions import Fraction

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gemma-webgpu-engine_amd", "csrc")
HEADER = os.path.join(CSRC, "gs_exp2_table.h")
BOUND = 4.2e-10


def header_constants():
    text = open(HEADER).read()
    table_text = text[text.index("GS_EXP2_TABLE_256"):text.index("// Taylor")]
    table = [float.fromhex(h) for h in re.findall(r"0x[0-9a-f.]+p[-+]\d+", table_text)]
    consts = {name: float.fromhex(v) for name, v in re.findall(r"#define (GS_\w+) (0x[0-9a-f.]+p[-+]\d+)", text)}
    return table, consts


def test_header_is_what_the_generator_writes():
    sys.path.insert(0, CSRC)
    try:
        import gen_exp2_table
    finally:
        sys.path.remove(CSRC)
    assert open(HEADER).read() == gen_exp2_table.render()


def test_table_entries_are_correctly_rounded():
    getcontext().prec = 60
    table, consts = header_constants()
    assert len(table) == 256
    for j, t in enumerate(table):
        exact = Decimal(2) ** (Decimal(j) / Decimal(256))  # a different route than exp(j ln2 / 256)
        # correctly rounded: every entry lies in [1, 2), where binary64 spacing is 2^-52
        assert 1.0 <= t < 2.0
        assert abs(Decimal(t) - exact) <= Decimal(2) ** -53, j
    ln2 = Decimal(2).ln()
    assert consts["GS_EXP2_256_C1"] == float(ln2 / 256)
    assert consts["GS_EXP2_256_C2"] == float((ln2 / 256) ** 2 / 2)
    assert consts["GS_256_LOG2E"] == float(256 / ln2)


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def exp2_256(y, table, c1, c2):
    n = round(y)  # binary64 rint: ties to even, as Python rounds floats
    s = y - n     # exact: |y| < 2^52
    p = fma(s, fma(s, c2, c1), 1.0)
    return float(Fraction(table[n & 255]) * Fraction(p)) * 2.0 ** (n >> 8)


def max_rel_error(c2):
    getcontext().prec = 40
    table, consts = header_constants()
    c1 = consts["GS_EXP2_256_C1"]
    worst = 0.0
    ys = []
    for n in (-22160, -5000, -1, 0, 255, 256, -257):
        for k in range(-50, 51):
            ys.append(n + k / 100.0)          # s across [-1/2, 1/2]
        ys += [n + 0.5 - 2.0 ** -40, n - 0.5 + 2.0 ** -40]
    for y in ys:
        got = exp2_256(y, table, c1, c2)
        exact = (Decimal(y) / 256 * Decimal(2).ln()).exp()
        worst = max(worst, float(abs((Decimal(got) - exact) / exact)))
    return worst


def test_exp2_256_relative_error_is_within_its_bound():
    _, consts = header_constants()
    err = max_rel_error(consts["GS_EXP2_256_C2"])
    assert err <= BOUND, err
    assert err >= 0.5 * BOUND  # the bound is the quadratic's truncation, and it is reached near |s| = 1/2


def test_the_bound_catches_a_dropped_term():
    """Without the s^2 term the error is three orders larger: the check above
    would fail on that mistake."""
    assert max_rel_error(0.0) > 100 * BOUND
