#!/usr/bin/env python3
"""Writes gs_exp2_table.h: the constants of the chunk scan's normaliser
exponential 2^(y/256) = 2^(j/256) * 2^k * e^(s ln2/256), |s| <= 1/2.

Every value is computed in 80-digit decimal arithmetic and rounded once to
binary64 (Python's float(Decimal) rounds correctly):
  GS_EXP2_TABLE_256   2^(j/256), j = 0..255
  GS_EXP2_256_C1..C4  Taylor coefficients (ln2/256)^k / k!, k = 1..4
  GS_256_LOG2E        256 / ln 2

usage: python gen_exp2_table.py [output path]   (default: next to this file)
"""
import os
import sys
from decimal import Decimal, getcontext

getcontext().prec = 80


def hexf(x: Decimal) -> str:
    h = float(x).hex()  # '0x1.62e42fefa39efp-9'
    mant, exp = h.split("p")
    return f"{mant}p{exp}"


def render() -> str:
    ln2 = Decimal(2).ln()
    table = [hexf((ln2 * j / 256).exp()) for j in range(256)]
    lines = [
        "// 2^(j/256), j = 0..255, each correctly rounded to binary64 (generated from",
        "// 80-digit decimal arithmetic by gen_exp2_table.py). Used by the streaming",
        "// normaliser of the chunk scan.",
        "#pragma once",
        "#define GS_EXP2_TABLE_256 \\",
    ]
    for i in range(0, 256, 4):
        row = ", ".join(table[i:i + 4])
        lines.append(f"  {row}{', ' if i + 4 < 256 else ''}\\" if i + 4 < 256 else f"  {row}")
    c = ln2 / 256
    lines += [
        "",
        "// Taylor coefficients (ln2/256)^k / k!, k = 1..4, and 256 / ln2",
        f"#define GS_EXP2_256_C1 {hexf(c)}",
        f"#define GS_EXP2_256_C2 {hexf(c * c / 2)}",
        f"#define GS_EXP2_256_C3 {hexf(c * c * c / 6)}",
        f"#define GS_EXP2_256_C4 {hexf(c * c * c * c / 24)}",
        f"#define GS_256_LOG2E {hexf(256 / ln2)}",
        "",
    ]
    return "\n".join(lines)


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                             "gs_exp2_table.h")
    with open(out, "w") as f:
        f.write(render())
