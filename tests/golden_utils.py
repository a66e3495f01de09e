"""Helpers shared by the CPU and GPU parity tests: the golden fixtures and the exact-sum classification of
rotation mismatches."""

from __future__ import annotations

import glob
import os
from fractions import Fraction

import numpy as np

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture_names() -> list[str]:
    return sorted(os.path.splitext(os.path.basename(p))[0] for p in glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def load_fixture(name: str) -> dict:
    with np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"), allow_pickle=False) as data:
        out = {k: data[k] for k in data.files}
    out["M"], out["K"], out["N"], out["G"] = (int(v) for v in out["shape"])
    return out


def bf16_value(bits: int) -> Fraction:
    return Fraction(float(np.array([bits << 16], dtype=np.uint32).view(np.float32)[0]))


def fraction_to_bf16(v: Fraction) -> int:
    """Round an exact rational to bf16 (nearest, ties to even) with Python's exact Fraction arithmetic."""
    if v == 0:
        return 0
    sign = 0x8000 if v < 0 else 0
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = max(e - 7, -133)
    quantum = Fraction(2) ** q
    k = round(a / quantum)  # Fraction.__round__ rounds half to even
    value = k * quantum
    if value >= Fraction(2) ** 128:
        return sign | 0x7F80
    f = np.array([float(value)], dtype=np.float32)
    return sign | int(f.view(np.uint32)[0] >> 16)


def fraction_to_f32(v: Fraction) -> float:
    """Round an exact rational to fp32 (nearest, ties to even) with Python's exact Fraction arithmetic."""
    if v == 0:
        return 0.0
    sign = -1.0 if v < 0 else 1.0
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = max(e - 23, -149)
    quantum = Fraction(2) ** q
    k = round(a / quantum)  # Fraction.__round__ rounds half to even
    value = k * quantum
    if value >= Fraction(2) ** 128:
        return sign * float("inf")
    return sign * float(np.float32(float(value)))


def hadamard_column_signs(group: int, j: int) -> np.ndarray:
    """Signs of column j of the unnormalised regular Hadamard (-1 where an odd number of base-4 digit pairs sum
    to 3)."""
    i = np.arange(group)
    neg = np.zeros(group, dtype=bool)
    n = 0
    while 4**n < group:
        n += 1
    for t in range(n):
        neg ^= (((i >> (2 * t)) & 3) + ((j >> (2 * t)) & 3)) == 3
    return np.where(neg, -1, 1)


def exact_rotation(x_bits: np.ndarray, row: int, col: int, group: int) -> Fraction:
    """The exact value of (x @ blockdiag(H))[row, col] as a Fraction."""
    g0 = (col // group) * group
    n = 0
    while 4**n < group:
        n += 1
    signs = hadamard_column_signs(group, col - g0)
    total = Fraction(0)
    for i in range(group):
        b = int(x_bits[row, g0 + i])
        if b & 0x7FFF:
            total += signs[i] * bf16_value(b)
    return total / (2**n)


def classify_rotation_mismatches(x_bits: np.ndarray, xr_exact: np.ndarray, xr_other: np.ndarray, group: int,
                                 limit: int = 2000) -> tuple[int, list]:
    """Compare an exactly rounded rotation with one whose sum was accumulated in fp32 (the reference's torch CPU
    GEMM). A mismatch is explained when (a) the exact value rounds to ``xr_exact`` and (b) ``xr_other`` is within
    the fp32 accumulation error bound (G * 2^-24 * sum |terms|) plus half a bf16 ulp of the exact value. Returns
    (number of mismatches, list of unexplained (row, col) positions)."""
    a = (np.asarray(xr_exact).astype(np.uint32) << 16).view(np.float32)
    b = (np.asarray(xr_other).astype(np.uint32) << 16).view(np.float32)
    where = np.argwhere(a != b)
    unexplained = []
    for row, col in where[:limit]:
        exact = exact_rotation(x_bits, row, col, group)
        if fraction_to_bf16(exact) != int(xr_exact[row, col]) and not (exact == 0 and a[row, col] == 0):
            unexplained.append((int(row), int(col), "exact rounding"))
            continue
        g0 = (col // group) * group
        terms = np.abs((np.asarray(x_bits[row, g0:g0 + group]).astype(np.uint32) << 16).view(np.float32))
        n = 0
        while 4**n < group:
            n += 1
        bound = Fraction(float(group * 2.0**-24 * float(terms.astype(np.float64).sum()) / 2**n))
        other = Fraction(float(b[row, col]))
        half_ulp = Fraction(abs(float(b[row, col]))) * Fraction(1, 2**8) + Fraction(2) ** -134
        if abs(other - exact) > bound + half_ulp:
            unexplained.append((int(row), int(col), "beyond fp32 accumulation bound"))
    return len(where), unexplained


def within_fp32_sum_bound(got: np.ndarray, ref: np.ndarray, x: np.ndarray, d: np.ndarray) -> bool:
    """Whether bf16 results ``got`` of fp32 sums of K products (rows of x [M, K] against rows of d [R, K], as float
    values) are within the error of some summation order of the exactly rounded sums ``ref``: recursive fp32 summation
    in any order is within K 2^-24 sum_k |x_k d_k| of the exact sum, and each result is rounded to bf16 once (2^-7 of
    |ref| covers both roundings). Near cancellations (an exact sum far below its terms) can only be held to that; a
    bitwise-fraction check covers the typical element."""
    x = np.asarray(x, dtype=np.float64)
    d = np.asarray(d, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = np.abs(ref) * 2.0**-7 + x.shape[1] * 2.0**-24 * (np.abs(x) @ np.abs(d).T)
    return bool((np.abs(np.asarray(got, dtype=np.float64) - ref) <= bound).all())
