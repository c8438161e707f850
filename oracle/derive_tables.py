"""Exact derivation of the NOVA F(6,3) transform tables (test infrastructure).

This file belongs to the CPU oracle. It is used only by the tests and by the
oracle itself; the product library carries its own copy of the resulting fp32
bit patterns and a CPU test checks that both copies equal what this module
derives.

The reference hard-codes three fp32 tables for the interpolation points
{0, +-3/5, +-1, +-7/6, inf} (/root/reference/csrc/nova_winograd.hip:68-97):

* ``A`` (6x8): row r holds the r-th powers of the finite points; the infinity
  column is the unit vector e_5.
* ``G`` (8x3): row i is [1, a_i, a_i^2] / N(a_i) with
  N(a_i) = prod_{j != i, j finite} (a_i - a_j); the infinity row is [0, 0, 1].
* ``B`` (8x8): column i holds the coefficients (power 0..7) of the monic
  polynomial prod_{j != i, j finite} (x - a_j); the infinity column holds the
  coefficients of prod_{j finite} (x - a_j).

With these tables, ``A [(G w G^T) * (B^T d B)] A^T`` equals the 6x6 valid
correlation of an 8x8 patch ``d`` with a 3x3 filter ``w`` exactly (checked in
tests/test_oracle.py with rational arithmetic).

The reference stores decimal literals (10 significant digits) that the
compiler rounds to fp32; the exact rationals below round to the same fp32
values (also checked), then A and B are rounded once more to fp16 exactly as
the reference's constant upload does (nova_winograd.hip:103-131).
"""

from fractions import Fraction as F
import struct

POINTS = [F(0), F(3, 5), F(-3, 5), F(1), F(-1), F(7, 6), F(-7, 6)]  # + infinity
N_PTS = 8  # n = m + r - 1 = 6 + 3 - 1


def _poly_from_roots(roots):
    """Coefficients (power 0..deg) of prod (x - r)."""
    coeffs = [F(1)]
    for r in roots:
        nxt = [F(0)] * (len(coeffs) + 1)
        for i, c in enumerate(coeffs):
            nxt[i + 1] += c
            nxt[i] -= r * c
        coeffs = nxt
    return coeffs


def exact_tables():
    """Return (A 6x8, B 8x8, G 8x3) as lists of Fractions."""
    fin = POINTS
    A = [[F(0)] * N_PTS for _ in range(6)]
    for r in range(6):
        for i, a in enumerate(fin):
            A[r][i] = a ** r
    A[5][7] = F(1)

    G = [[F(0)] * 3 for _ in range(N_PTS)]
    for i, a in enumerate(fin):
        n = F(1)
        for j, b in enumerate(fin):
            if j != i:
                n *= (a - b)
        G[i] = [F(1) / n, a / n, a * a / n]
    G[7] = [F(0), F(0), F(1)]

    B = [[F(0)] * N_PTS for _ in range(N_PTS)]
    for i in range(7):
        coeffs = _poly_from_roots([b for j, b in enumerate(fin) if j != i])
        for p, c in enumerate(coeffs):
            B[p][i] = c
    coeffs = _poly_from_roots(fin)
    for p, c in enumerate(coeffs):
        B[p][7] = c
    return A, B, G


def _round_fraction(x, mant_bits, min_exp, max_exp):
    """Round a Fraction to the nearest binary float with ``mant_bits`` bits of
    significand (including the hidden bit), ties to even.  Returns a Fraction.
    ``min_exp`` is the exponent of the smallest normal; subnormals keep the
    fixed quantum 2**(min_exp - mant_bits + 1)."""
    if x == 0:
        return F(0)
    sign = -1 if x < 0 else 1
    ax = abs(x)
    e = ax.numerator.bit_length() - ax.denominator.bit_length()
    if F(2) ** e > ax:
        e -= 1
    while F(2) ** (e + 1) <= ax:
        e += 1
    e = max(e, min_exp)
    quantum = F(2) ** (e - mant_bits + 1)
    q = ax / quantum
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > F(1, 2) or (rem == F(1, 2) and fl % 2 == 1):
        fl += 1
    val = fl * quantum
    if val >= F(2) ** (max_exp + 1):
        raise OverflowError("value out of range")
    return sign * val


def to_f32(x):
    """Exact round-to-nearest-even of a Fraction to fp32 (returns a Python float)."""
    return float(_round_fraction(F(x), 24, -126, 127))


def to_f16(x):
    """Exact round-to-nearest-even of a Fraction/float to fp16 (returns a Python float)."""
    return float(_round_fraction(F(x), 11, -14, 15))


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def f16_bits(v):
    return struct.unpack("<H", struct.pack("<e", v))[0]


def fp32_tables():
    """(A, B, G) rounded to fp32, plus (Ah, Bh) = fp16(fp32(.)) as floats."""
    A, B, G = exact_tables()
    A32 = [[to_f32(v) for v in row] for row in A]
    B32 = [[to_f32(v) for v in row] for row in B]
    G32 = [[to_f32(v) for v in row] for row in G]
    Ah = [[to_f16(v) for v in row] for row in A32]
    Bh = [[to_f16(v) for v in row] for row in B32]
    return A32, B32, G32, Ah, Bh


def c_initializer(table, fmt="f32"):
    """Render a table as a C initializer of hex-float literals."""
    rows = []
    for row in table:
        if fmt == "f32":
            rows.append("{" + ", ".join(float.hex(v) + "f" for v in row) + "}")
        else:
            rows.append("{" + ", ".join(float.hex(v) for v in row) + "}")
    return "{\n    " + ",\n    ".join(rows) + "\n}"


if __name__ == "__main__":
    A32, B32, G32, Ah, Bh = fp32_tables()
    print("A =", c_initializer(A32))
    print("B =", c_initializer(B32))
    print("G =", c_initializer(G32))
    print("Ah =", c_initializer(Ah))
    print("Bh =", c_initializer(Bh))
