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


def _bf16_f64(bits) -> np.ndarray:
    return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def bf16_half_ulp(bits) -> np.ndarray:
    """Half a bf16 unit in the last place at each value's binade (2^(e-8) for |v| in [2^e, 2^(e+1)); the subnormal
    spacing below 2^-126). Rounding v to bf16 moves it by at most this at the rounded value's binade."""
    v = np.abs(_bf16_f64(bits))
    e = np.floor(np.log2(np.maximum(v, 2.0**-126)))
    return 2.0 ** (e - 8)


def ulp_steps(a_bits, b_bits) -> np.ndarray:
    """Distance between two bf16 arrays counted in representable values (0: bitwise equal, 1: neighbours)."""
    def ordered(bits):
        b = np.asarray(bits).astype(np.int64)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)

    return np.abs(ordered(a_bits) - ordered(b_bits))


def composition_error_bound(y_bits, lowrank_bits, bias_bits, composed_bits, fused_bits) -> np.ndarray:
    """The largest |fused - composed| that rounding alone allows, elementwise.

    ``composed`` is the reference's composition ``Int8RotLinear(x) + LowRankLinear(x) + bias`` in bf16 tensor
    arithmetic (transformer.py:57-58; each ``+`` rounds to bf16): ``rb(rb(y8 + lr) + bias)`` with ``y_bits`` =
    rb(y8) the INT8 layer's output and ``lowrank_bits`` = rb(lr) the low-rank layer's (either term may be absent).
    ``fused`` rounds the same exact sum ``y8 + lr + bias`` once. Each rounding to bf16 moves a value by at most half
    a unit at its rounded magnitude, so the two results differ by at most the sum of those half units; the factor
    1 + 2^-6 covers the fp32 addition ahead of each bf16 rounding. A dropped, doubled, negated or transposed term
    moves results by far more on some elements."""
    terms = bf16_half_ulp(y_bits) + bf16_half_ulp(composed_bits) + bf16_half_ulp(fused_bits)
    if lowrank_bits is not None:
        terms = terms + bf16_half_ulp(lowrank_bits)
        if bias_bits is not None:  # the intermediate rb(y + lr) before the bias is added
            s = (_bf16_f64(y_bits) + _bf16_f64(lowrank_bits)).astype(np.float32)
            t1 = ((s.view(np.uint32) + 0x7FFF + ((s.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
            terms = terms + bf16_half_ulp(t1)
    return terms * (1.0 + 2.0**-6)


def check_against_composition(got_bits, y_bits, lowrank_bits, bias_bits, composed_bits, extra=None,
                              min_share: float = 0.995) -> None:
    """The fused extension's bar against the reference's composition, elementwise: every element within
    ``composition_error_bound`` (+ ``extra``, a device's own summation slack), at least ``min_share`` of the
    elements within one bf16 step of the composition, and max |Δ| / max |composed| <= 1e-2."""
    got = _bf16_f64(got_bits)
    comp = _bf16_f64(composed_bits)
    bound = composition_error_bound(y_bits, lowrank_bits, bias_bits, composed_bits, got_bits)
    if extra is not None:
        bound = bound + extra
    bad = np.abs(got - comp) > bound
    assert not bad.any(), f"{int(bad.sum())} elements beyond the rounding bound, first at {np.argwhere(bad)[0]}"
    share = float((ulp_steps(got_bits, composed_bits) <= 1).mean())
    assert share >= min_share, share
    assert np.abs(got - comp).max() / np.abs(comp).max() <= 1e-2


def device_lowrank_slack(x_bits, down_bits, u_ref_bits, up_bits, y_bits, bias_bits=None) -> np.ndarray:
    """What fp32 accumulation on the device may add to ``composition_error_bound``, elementwise: the device's u
    (K products summed in fp32, rounded to bf16) is within 4 half units of the oracle's exactly rounded u plus
    K 2^-24 sum_k |x_k d_k| (``within_fp32_sum_bound``), and the epilogue sums y8, the r low-rank products and the
    bias in fp32 ((r + 2) 2^-24 of the sum of their magnitudes)."""
    x = _bf16_f64(x_bits)
    d = _bf16_f64(down_bits)
    u = _bf16_f64(u_ref_bits)
    up = np.abs(_bf16_f64(up_bits))
    du = 4 * bf16_half_ulp(u_ref_bits) + x.shape[1] * 2.0**-24 * (np.abs(x) @ np.abs(d).T)
    mag = np.abs(_bf16_f64(y_bits)) * (1 + 2.0**-7) + (np.abs(u) + du) @ up.T
    if bias_bits is not None:
        mag = mag + np.abs(_bf16_f64(bias_bits))[None, :]
    return du @ up.T + (u.shape[1] + 2) * 2.0**-24 * mag * 1.01
