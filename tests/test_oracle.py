"""The oracle pinned: against the reference's own golden vectors (tests/golden, written from the reference's
``_forward_torch``), closed forms, brute force in exact rational arithmetic, and planted mistakes that these checks
must catch. CPU only."""

from __future__ import annotations

import itertools
from fractions import Fraction

import numpy as np
import pytest

from golden_utils import (check_against_composition, classify_rotation_mismatches, composition_error_bound,
                          fixture_names, fraction_to_bf16, fraction_to_f32, load_fixture, ulp_steps)

FIXTURES = fixture_names()


def test_fixtures_present():
    assert len(FIXTURES) >= 7, FIXTURES


# ----------------------------------------------------------------------------------------- Hadamard (int8.py:100-119)


@pytest.mark.parametrize("group", [4, 16, 64, 256, 1024])
def test_regular_hadamard_closed_form(oracle_lib, group):
    h = oracle_lib.regular_hadamard(group)
    np.testing.assert_array_equal(h, oracle_lib.regular_hadamard_c(group))
    np.testing.assert_allclose(h @ h.T, np.eye(group), atol=1e-12)
    np.testing.assert_array_equal(h, h.T)
    np.testing.assert_allclose(h.sum(axis=1), np.ones(group), atol=1e-12)  # "rows sum to one"
    assert set(np.unique(np.abs(h))) == {group ** -0.5}


@pytest.mark.parametrize("group", [2, 8, 32, 128, 512])
def test_regular_hadamard_rejects_non_powers_of_four(oracle_lib, group):
    with pytest.raises(ValueError):
        oracle_lib.regular_hadamard(group)
    with pytest.raises(ValueError):
        oracle_lib.regular_hadamard_c(group)


@pytest.mark.parametrize("group", [256, 1024, 4096])
def test_hadamard_factors_rebuild_the_rotation(oracle_lib, group):
    ga, gb = oracle_lib.hadamard_factors(group)
    assert ga >= 16 and gb >= 16
    np.testing.assert_array_equal(np.kron(oracle_lib.regular_hadamard(ga), oracle_lib.regular_hadamard(gb)),
                                  oracle_lib.regular_hadamard(group))


def test_small_groups_have_no_factors(oracle_lib):
    assert oracle_lib.hadamard_factors(16) is None and oracle_lib.hadamard_factors(64) is None


# --------------------------------------------------------------------------------- the rotation (int8.py:176)


def _bits(values) -> np.ndarray:
    return oracle_lib_f32_to_bf16(np.asarray(values, dtype=np.float32))


def oracle_lib_f32_to_bf16(a):
    from oracle import oracle

    return oracle.f32_to_bf16(a)


@pytest.mark.parametrize("group", [4, 16, 64])
def test_rotation_is_the_exact_sum_rounded_once(oracle_lib, group):
    """Brute force in exact rational arithmetic, on inputs spanning up to ~250 binades, with zeros and signs."""
    rng = np.random.default_rng(group)
    rows = []
    for _ in range(6):
        mags = rng.standard_normal(group) * np.exp2(rng.integers(-60, 60, size=group).astype(np.float64))
        mags[rng.random(group) < 0.1] = 0.0
        rows.append(mags)
    rows.append(np.exp2(rng.integers(-120, 120, size=group).astype(np.float64)) * rng.choice([-1, 1], size=group))
    x = _bits(np.array(rows, dtype=np.float64).astype(np.float32))
    got = oracle_lib.rotate(x, group, force_exact=True)
    h = oracle_lib.regular_hadamard(group)
    for r in range(x.shape[0]):
        xv = [Fraction(float(v)) for v in oracle_lib.bf16_to_f32(x[r])]
        for j in range(group):
            exact = sum((xv[i] * Fraction(h[i, j]) for i in range(group)), Fraction(0))
            assert fraction_to_bf16(exact) == int(got[r, j]), (r, j)


def _exact_rotation_ints(xv: np.ndarray, group: int, signs: np.ndarray) -> list[Fraction]:
    """The exact sums of one bf16 row against the +-1 signs of the regular Hadamard, in Python integers (an integer
    dot product, not a butterfly), scaled back by the row's smallest power of two and the 2^-n normalisation."""
    m, e = np.frexp(xv.astype(np.float64))  # xv = m * 2^e, m with at most 8 significant bits
    mant = np.round(m * 256).astype(np.int64)
    nz = mant != 0
    e_min = int(e[nz].min()) - 8 if nz.any() else 0
    ints = np.array([int(v) << int(ei - 8 - e_min) if v else 0 for v, ei in zip(mant, e)], dtype=object)
    n = (group.bit_length() - 1) // 2
    sums = ints.dot(signs.astype(object))
    return [Fraction(int(t)) * Fraction(2) ** (e_min - n) for t in sums]


@pytest.mark.parametrize("group,rows", [(256, 3), (1024, 2), (4096, 1)])
def test_rotation_large_groups_exact_integer_sums(oracle_lib, group, rows):
    """Groups that span whole 1024-element tiles: the exact sums as integer dot products (any magnitude: Python
    integers), one row spanning ~250 binades (the oracle's wide accumulator) and narrow rows (its float64 path)."""
    rng = np.random.default_rng(group + 7)
    data = [np.exp2(rng.integers(-120, 120, size=group).astype(np.float64)) * rng.choice([-1, 1], size=group)]
    for _ in range(rows - 1):
        data.append(rng.standard_normal(group) * 4.0)
    x = _bits(np.array(data, dtype=np.float64).astype(np.float32))
    signs = np.sign(oracle_lib.regular_hadamard(group)).astype(np.int64)
    got = oracle_lib.rotate(x, group)
    got_exact = oracle_lib.rotate(x, group, force_exact=True)
    for r in range(x.shape[0]):
        exact = _exact_rotation_ints(oracle_lib.bf16_to_f32(x[r]), group, signs)
        want = np.array([fraction_to_bf16(v) for v in exact], dtype=np.uint16)
        np.testing.assert_array_equal(got_exact[r], want)
        np.testing.assert_array_equal(got[r], want)


def test_rotation_rounds_ties_to_even(oracle_lib):
    # G=4: out_0 = (x0 + x1 + x2 - x3) / 2. (1 + 2^-8)/2 = 0.5 + 2^-9 is the midpoint between 0.5 (even) and
    # 0.5 + 2^-8; (1 + 3*2^-8)/2 is the midpoint between 0.5 + 2^-8 (odd) and 0.5 + 2^-7 (even).
    x = _bits([[1.0, 2.0**-8, 0.0, 0.0], [1.0, 3 * 2.0**-8, 0.0, 0.0]])
    out = oracle_lib.bf16_to_f32(oracle_lib.rotate(x, 4, force_exact=True))
    assert out[0, 0] == 0.5 and out[1, 0] == 0.5 + 2.0**-7
    out_fast = oracle_lib.bf16_to_f32(oracle_lib.rotate(x, 4))
    np.testing.assert_array_equal(out, out_fast)


@pytest.mark.parametrize("name", FIXTURES)
def test_rotation_fast_path_equals_exact_path(oracle_lib, name):
    f = load_fixture(name)
    x = f["x"][:16]
    np.testing.assert_array_equal(oracle_lib.rotate(x, f["G"]), oracle_lib.rotate(x, f["G"], force_exact=True))


# ------------------------------------------------------------------------------ quantization (int8.py:177-178)


def test_quantize_zero_row_and_half_even_ties(oracle_lib):
    # Row 0 all zero: clamp_min(1e-12) / 127. Row 1: amax 127 gives sx == 1 exactly, so xr / sx hits the halves.
    xr = _bits([[0.0] * 8, [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5]])
    sx, xq = oracle_lib.quantize(xr)
    assert sx[0] == np.float32(np.float32(1e-12) / np.float32(127.0)) and not xq[0].any()
    assert sx[1] == 1.0
    assert xq[1].tolist() == [127, 2, 4, -2, -4, 0, 2, 0]


def test_quantize_divides_rather_than_multiplying_by_the_reciprocal(oracle_lib):
    # A value whose true quotient rounds differently from a * (1/s): search small integers for one.
    found = None
    for amax_q in range(100, 3000):
        amax = np.float32(amax_q) * np.float32(2.0**-7)
        s = np.float32(amax / np.float32(127.0))
        inv = np.float32(np.float32(1.0) / s)
        for num in range(1, 400):
            a = np.float32(num) * np.float32(2.0**-7)
            if a > amax:
                break
            if np.rint(np.float32(a / s)) != np.rint(np.float32(a * inv)):
                found = (amax, a)
                break
        if found:
            break
    assert found, "no case separating division from reciprocal multiplication"
    amax, a = found
    xr = _bits([[amax, a]])
    sx, xq = oracle_lib.quantize(xr)
    assert xq[0, 1] == np.rint(np.float32(a / sx[0]))


# ---------------------------------------------- the reference's GPU-kernel arithmetic (int8.py:194-262): fp32, 1/s
# No golden vectors exist for it (the reference's Triton kernels need CUDA): the restatement is pinned by exact
# arithmetic and by the cases that separate it from the torch path.


@pytest.mark.parametrize("group", [4, 16, 64])
def test_rotation_f32_is_the_exact_sum_rounded_once(oracle_lib, group):
    """Brute force in exact rational arithmetic on inputs spanning up to ~250 binades, both summation paths."""
    rng = np.random.default_rng(100 + group)
    rows = []
    for _ in range(5):
        mags = rng.standard_normal(group) * np.exp2(rng.integers(-60, 60, size=group).astype(np.float64))
        mags[rng.random(group) < 0.1] = 0.0
        rows.append(mags)
    rows.append(rng.standard_normal(group) * 3.0)  # a narrow span: the float64 path
    x = _bits(np.array(rows, dtype=np.float64).astype(np.float32))
    got_exact = oracle_lib.rotate_f32(x, group, force_exact=True)
    got_fast = oracle_lib.rotate_f32(x, group)
    h = oracle_lib.regular_hadamard(group)
    for r in range(x.shape[0]):
        xv = [Fraction(float(v)) for v in oracle_lib.bf16_to_f32(x[r])]
        for j in range(group):
            exact = sum((xv[i] * Fraction(h[i, j]) for i in range(group)), Fraction(0))
            want = fraction_to_f32(exact)
            assert float(got_exact[r, j]) == want, (r, j)
            assert float(got_fast[r, j]) == want, (r, j)


def test_rotation_f32_rounds_ties_to_even(oracle_lib):
    # G=4: out_0 = (x0 + x1 + x2 - x3) / 2. (1 + 2^-24)/2 = 0.5 + 2^-25 is the midpoint between 0.5 (even) and
    # 0.5 + 2^-24; (1 + 3*2^-24)/2 is the midpoint between 0.5 + 2^-24 (odd) and 0.5 + 2^-23 (even).
    x = _bits([[1.0, 2.0**-24, 0.0, 0.0], [1.0, 3 * 2.0**-24, 0.0, 0.0]])
    for exact in (True, False):
        out = oracle_lib.rotate_f32(x, 4, force_exact=exact)
        assert out[0, 0] == np.float32(0.5) and out[1, 0] == np.float32(0.5 + 2.0**-23)


@pytest.mark.parametrize("name", FIXTURES)
def test_rotation_f32_and_bf16_agree_after_bf16_rounding(oracle_lib, name):
    """Rounding the fp32 rotation to bf16 gives the bf16 rotation except where the fp32 rounding lands exactly on a
    bf16 midpoint (a double rounding), which the exact sums show."""
    f = load_fixture(name)
    x = f["x"][:16]
    f32 = oracle_lib.rotate_f32(x, f["G"])
    b16 = oracle_lib.rotate(x, f["G"])
    again = oracle_lib.f32_to_bf16(f32)
    bad = again != b16
    ties = (f32.view(np.uint32) & 0xFFFF) == 0x8000
    assert not (bad & ~ties).any()


def test_quantize_recip_multiplies_by_the_reciprocal(oracle_lib):
    """The case that separates a * (1/s) from a / s (the torch path's division): the GPU-kernel quantization takes
    the reciprocal product."""
    found = None
    for amax_q in range(100, 3000):
        amax = np.float32(amax_q) * np.float32(2.0**-7)
        s = np.float32(amax / np.float32(127.0))
        inv = np.float32(np.float32(1.0) / s)
        for num in range(1, 400):
            a = np.float32(num) * np.float32(2.0**-7)
            if a > amax:
                break
            if np.rint(np.float32(a / s)) != np.rint(np.float32(a * inv)):
                found = (amax, a)
                break
        if found:
            break
    assert found
    amax, a = found
    sx, xq = oracle_lib.quantize_recip(np.array([[amax, a]], dtype=np.float32))
    inv = np.float32(np.float32(1.0) / sx[0])
    assert xq[0, 1] == np.rint(np.float32(a * inv)) and xq[0, 1] != np.rint(np.float32(a / sx[0]))


def test_quantize_recip_zero_row_ties_and_extremes(oracle_lib):
    # zero row: scale 1e-12 / 127 and zero codes; amax 127 gives s = 1 and inv = 1, so the halves tie to even
    xr = np.array([[0.0] * 8, [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5]], dtype=np.float32)
    sx, xq = oracle_lib.quantize_recip(xr)
    assert sx[0] == np.float32(np.float32(1e-12) / np.float32(127.0)) and not xq[0].any()
    assert sx[1] == 1.0 and xq[1].tolist() == [127, 2, 4, -2, -4, 0, 2, 0]
    # every nonzero row reaches +-127 at its absmax and no code leaves [-127, 127]
    f = load_fixture(FIXTURES[0])
    sx, xq = oracle_lib.quantize_recip(oracle_lib.rotate_f32(f["x"], f["G"]))
    assert (np.abs(xq.astype(np.int32)).max(axis=1) == 127).all()


def test_gpu_kernel_arithmetic_differs_from_the_torch_path(oracle_lib):
    """A planted swap of the two arithmetics is visible: on benchmark-like rows every scale and a few percent of the
    codes differ (each by one)."""
    inp = oracle_lib.make_inputs(64, 5120, 8, 256, outlier_frac=0.005, outlier_scale=30.0, seed=3)
    sx_t, xq_t = oracle_lib.quantize(oracle_lib.rotate(inp["x"], 256))
    sx_k, xq_k = oracle_lib.quantize_recip(oracle_lib.rotate_f32(inp["x"], 256))
    assert (sx_t != sx_k).mean() > 0.5
    diff = xq_t.astype(np.int32) - xq_k.astype(np.int32)
    assert 0.005 < (diff != 0).mean() < 0.2 and np.abs(diff).max() == 1


# ------------------------------------------------------------------------------------ GEMM and epilogue (int8.py:179)


def test_int8_gemm_is_the_exact_integer_product(oracle_lib):
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, size=(37, 300), dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, size=(29, 300), dtype=np.int64).astype(np.int8)
    np.testing.assert_array_equal(oracle_lib.int8_gemm(a, b), a.astype(np.int64) @ b.astype(np.int64).T)
    big = np.full((1, 140000), 127, dtype=np.int8)
    with pytest.raises(OverflowError):
        oracle_lib.int8_gemm(big, big)


def _rn32(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp32 (ties to even), by exact arithmetic."""
    if v == 0:
        return v
    e = abs(v).numerator.bit_length() - abs(v).denominator.bit_length()
    if Fraction(2) ** e > abs(v):
        e -= 1
    quantum = Fraction(2) ** (e - 23)
    return round(v / quantum) * quantum


def test_epilogue_order_is_left_to_right(oracle_lib):
    """int8.py:179 evaluates ``(acc * sx) * wscale``: two fp32 roundings in that order. Search for operands where
    the other association ``acc * (sx * wscale)`` rounds to a different bf16, and check the oracle takes the
    reference's order (computed here in exact rational arithmetic)."""
    rng = np.random.default_rng(9)
    n = 1 << 20
    acc = rng.integers(-2**22, 2**22, size=n).astype(np.int32)
    sx = rng.uniform(1e-3, 1e-1, size=n).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    a32 = acc.astype(np.float32)
    cand = np.nonzero(oracle_lib.f32_to_bf16((a32 * sx) * ws) != oracle_lib.f32_to_bf16(a32 * (sx * ws)))[0][:64]
    left, right, picked = [], [], []
    for i in cand:  # confirm each candidate in exact rational arithmetic
        a, s_, w = Fraction(int(acc[i])), Fraction(float(sx[i])), Fraction(float(ws[i]))
        lv, rv = fraction_to_bf16(_rn32(_rn32(a * s_) * w)), fraction_to_bf16(_rn32(a * _rn32(s_ * w)))
        if lv != rv:
            picked.append(i)
            left.append(lv)
    assert picked, "no operands separate the two association orders"
    got = [int(oracle_lib.epilogue(acc[i:i + 1, None].copy(), sx[i:i + 1], ws[i:i + 1])[0, 0]) for i in picked]
    assert got == left


# -------------------------------------------------------------------------- pinned to the reference's own outputs


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_matches_reference_golden(oracle_lib, name):
    f = load_fixture(name)
    out = oracle_lib.convrot_linear(f["x"], f["qweight"], f["wscale"], f["G"])
    mismatches, unexplained = classify_rotation_mismatches(f["x"], out["xr"], f["xr"], f["G"])
    assert not unexplained, unexplained
    assert mismatches <= max(2, 1e-5 * out["xr"].size), mismatches
    np.testing.assert_array_equal(out["sx"], f["sx"])
    np.testing.assert_array_equal(out["xq"], f["xq"])
    np.testing.assert_array_equal(out["acc"], f["acc"])
    np.testing.assert_array_equal(out["y"], f["y"])


def test_composition_matches_reference_golden(oracle_lib):
    f = load_fixture("composition")
    np.testing.assert_array_equal(oracle_lib.lowrank_down(f["x"], f["down"]), f["u"])
    comp = oracle_lib.composition(f["y"], f["x"], f["down"], f["up"], f["bias"])
    np.testing.assert_array_equal(comp, f["y_composed"])


def _fused_case(oracle_lib, f, mistake=None):
    """The oracle's fused epilogue on the composition fixture, optionally with one planted mistake in its operands."""
    out = oracle_lib.convrot_linear(f["x"], f["qweight"], f["wscale"], f["G"])
    u = oracle_lib.lowrank_down(f["x"], f["down"])
    up, bias = f["up"], f["bias"]
    m, r = u.shape
    n = up.shape[0]
    if mistake == "bias_dropped":
        bias = None
    elif mistake == "lowrank_dropped":
        u = up = None
    elif mistake == "both_dropped":
        u = up = bias = None
    elif mistake == "up_transposed":  # up's [N, r] memory read as [r, N]
        up = np.ascontiguousarray(up.reshape(r, n).T)
    elif mistake == "u_transposed":
        u = np.ascontiguousarray(u.reshape(r, m).T)
    elif mistake == "half_rank":
        u, up = np.ascontiguousarray(u[:, : r // 2]), np.ascontiguousarray(up[:, : r // 2])
    elif mistake == "lowrank_negated":
        up = up ^ np.uint16(0x8000)
    elif mistake == "bias_doubled":
        bias = oracle_lib.f32_to_bf16(2 * oracle_lib.bf16_to_f32(bias))
    return oracle_lib.fused_epilogue(out["acc"], out["sx"], f["wscale"], u, up, bias)


def test_fused_definition_matches_the_reference_composition_elementwise(oracle_lib):
    """The fused extension y = bf16((acc*sx)*ws + u @ up^T + bias) against the reference's own bf16 composition
    Int8RotLinear(x) + LowRankLinear(x) + bias (transformer.py:57-58, written by the reference's modules): every
    element within the rounding bound of the composition's three roundings, >= 99.5 % within one bf16 step."""
    f = load_fixture("composition")
    fused = _fused_case(oracle_lib, f)
    check_against_composition(fused, f["y"], f["lowrank"], f["bias"], f["y_composed"])
    assert float((ulp_steps(fused, f["y_composed"]) <= 1).mean()) >= 0.998  # measured 99.85 %


@pytest.mark.parametrize("mistake", ["bias_dropped", "lowrank_dropped", "both_dropped", "up_transposed",
                                     "u_transposed", "half_rank", "lowrank_negated", "bias_doubled"])
def test_planted_fused_mistakes_fail_the_composition_bar(oracle_lib, mistake):
    f = load_fixture("composition")
    bad = _fused_case(oracle_lib, f, mistake)
    bound = composition_error_bound(f["y"], f["lowrank"], f["bias"], f["y_composed"], bad)
    beyond = int((np.abs(oracle_lib.bf16_to_f32(bad).astype(np.float64)
                         - oracle_lib.bf16_to_f32(f["y_composed"])) > bound).sum())
    share = float((ulp_steps(bad, f["y_composed"]) <= 1).mean())
    assert beyond >= 100 and share < 0.99, (beyond, share)
    with pytest.raises(AssertionError):
        check_against_composition(bad, f["y"], f["lowrank"], f["bias"], f["y_composed"])


# ------------------------------------------------------------------------ planted mistakes the checks must catch


def _mutant_linear(oracle_lib, f, mistake):
    """The oracle's arithmetic restated in numpy with one planted mistake."""
    g, n = f["G"], int(np.log2(f["G"]) // 2)
    x = oracle_lib.bf16_to_f32(f["x"]).astype(np.float64)
    h = oracle_lib.regular_hadamard(g)
    if mistake == "sign_rule":
        i = np.arange(g)
        neg = np.zeros((g, g), dtype=bool)
        for t in range(n):
            neg ^= ((((i[:, None] >> (2 * t)) & 3) + ((i[None, :] >> (2 * t)) & 3)) == 0)
        h = np.where(neg, -1.0, 1.0) / 2**n
    rot = (x.reshape(x.shape[0], -1, g) @ h).reshape(x.shape)
    xr = rot.astype(np.float32) if mistake == "no_bf16_rounding" else oracle_lib.bf16_to_f32(
        oracle_lib.f64_to_bf16(rot))
    sx = (np.maximum(np.abs(xr).max(axis=1), np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    xq = np.clip(np.rint((xr / sx[:, None]).astype(np.float32)), -127, 127)
    acc = (xq.astype(np.int64) @ f["qweight"].astype(np.int64).T).astype(np.float32)
    y = (acc * sx[:, None]) * f["wscale"][None, :]
    return oracle_lib.f32_to_bf16(y.astype(np.float32)), sx


@pytest.mark.parametrize("mistake", ["sign_rule", "no_bf16_rounding"])
def test_planted_mistakes_are_caught_by_the_golden_vectors(oracle_lib, mistake):
    caught = 0
    for name in ("cfg1_slice", "odd_tail", "cfg2_slice"):
        f = load_fixture(name)
        y, sx = _mutant_linear(oracle_lib, f, mistake)
        caught += int((y != f["y"]).sum()) + int((sx != f["sx"]).sum())
    assert caught > 0, mistake


def test_unplanted_restatement_agrees(oracle_lib):
    """The numpy restatement above, with no mistake planted, agrees with the golden vectors (so the mutants fail
    only because of their mistake)."""
    for name in ("cfg1_slice", "odd_tail"):
        f = load_fixture(name)
        y, sx = _mutant_linear(oracle_lib, f, None)
        np.testing.assert_array_equal(sx, f["sx"])
        np.testing.assert_array_equal(y, f["y"])


# -------------------------------------------------------------------- checkpoint quantizer (test_int8.py:31-36)


def test_quantize_weight_against_a_direct_float64_loop(oracle_lib):
    rng = np.random.default_rng(5)
    w = rng.standard_normal((6, 32)) * 0.02
    q, ws = oracle_lib.quantize_weight(w, 16)
    h = oracle_lib.regular_hadamard(16)
    for o, k0 in itertools.product(range(6), range(0, 32, 16)):
        for j in range(16):
            rot = sum(w[o, k0 + i] * h[i, j] for i in range(16))
            amax = max(abs(sum(w[o, kk0 + i] * h[i, jj] for i in range(16)))
                       for kk0 in range(0, 32, 16) for jj in range(16))
            assert abs(float(ws[o]) - amax / 127.0) <= 1e-7 * amax
            assert int(q[o, k0 + j]) == int(np.clip(np.round(rot / (amax / 127.0)), -127, 127))


def test_lowrank_up_matches_reference_golden(oracle_lib):
    """The low-rank branch `up(down(x))` written by the reference's own bf16 modules (the composition fixture):
    from the golden u, the oracle's exactly rounded sum agrees within one bf16 ulp (torch's CPU bf16 GEMM sums in
    fp32 in its own order) and bitwise on almost every element."""
    f = load_fixture("composition")
    got = oracle_lib.bf16_to_f32(oracle_lib.lowrank_up(f["u"], f["up"]))
    ref = oracle_lib.bf16_to_f32(f["lowrank"])
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0**-7).all()
    assert (got == ref).mean() > 0.99


def test_lowrank_up_planted_transpose_is_caught(oracle_lib):
    """A transposed operand (u @ up instead of u @ up^T on a square case) must not pass the golden check."""
    f = load_fixture("composition")
    up = f["up"][:32]  # square 32 x 32 slice
    right = oracle_lib.bf16_to_f32(oracle_lib.lowrank_up(f["u"], up))
    wrong = oracle_lib.bf16_to_f32(oracle_lib.f64_to_bf16(
        oracle_lib.bf16_to_f32(f["u"]).astype(np.float64) @ oracle_lib.bf16_to_f32(up).astype(np.float64)))
    ref = oracle_lib.bf16_to_f32(f["lowrank"])[:, :32]
    assert (np.abs(right - ref) <= np.abs(ref) * 2.0**-7).all()
    assert not (np.abs(wrong - ref) <= np.abs(ref) * 2.0**-7).all()


# ------------------------------------------------------------------------------------- feed-forward activation


def test_gelu_tanh_matches_torch_on_every_bf16_value(oracle_lib):
    """The oracle's activation against torch's own `gelu(approximate="tanh")` (the reference's activation module) on
    every finite bf16 value: equal except where torch's fp32 tanh returns exactly -1 for an argument whose correctly
    rounded tanh is the next float up (a few values near x = -5, outputs of order 1e-7 against 0)."""
    import torch

    bits = np.arange(65536, dtype=np.uint16)
    bits = bits[np.isfinite(oracle_lib.bf16_to_f32(bits))]
    ours = oracle_lib.gelu_tanh(bits)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    theirs = torch.nn.functional.gelu(x, approximate="tanh").view(torch.int16).numpy().view(np.uint16)
    diff = ours != theirs
    assert diff.sum() <= 8
    assert np.abs(oracle_lib.bf16_to_f32(ours[diff]) - oracle_lib.bf16_to_f32(theirs[diff])).max(initial=0) < 1e-6


def test_gelu_tanh_closed_forms(oracle_lib):
    """Special values fixed by the formula: gelu(0) = 0, gelu(x) -> x for large x and -> 0 for very negative x, and
    gelu(1) = 0.5 (1 + tanh(sqrt(2/pi) * 1.044715)) = 0.8411920... (bf16 0.83984375)."""
    x = oracle_lib.f32_to_bf16(np.array([0.0, 1.0, 30.0, -30.0, 3.0e38], dtype=np.float32))
    g = oracle_lib.bf16_to_f32(oracle_lib.gelu_tanh(x))
    assert g[0] == 0.0 and g[2] == 30.0 and g[3] == 0.0 and g[4] == oracle_lib.bf16_to_f32(x[4:5])[0]
    exact = 0.5 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * 1.044715))
    assert g[1] == oracle_lib.bf16_to_f32(oracle_lib.f64_to_bf16(np.array([exact])))[0]


def test_gelu_tanh_planted_mistake_is_caught(oracle_lib):
    """A dropped cubic term (gelu with tanh(sqrt(2/pi) x)) fails the comparison with torch."""
    import torch

    rng = np.random.default_rng(3)
    bits = oracle_lib.f32_to_bf16((rng.standard_normal(4096) * 3).astype(np.float32))
    x = oracle_lib.bf16_to_f32(bits).astype(np.float64)
    wrong = oracle_lib.f64_to_bf16(0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * x)))
    theirs = torch.nn.functional.gelu(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16),
                                      approximate="tanh").view(torch.int16).numpy().view(np.uint16)
    assert (wrong != theirs).sum() > 100
    ours = oracle_lib.gelu_tanh(bits)
    assert np.abs(oracle_lib.bf16_to_f32(ours) - oracle_lib.bf16_to_f32(theirs)).max() < 1e-6


def test_silu_matches_torch_on_every_bf16_value(oracle_lib):
    """The oracle's SiLU against torch's own `silu` on every finite bf16 value."""
    import torch

    bits = np.arange(65536, dtype=np.uint16)
    bits = bits[np.isfinite(oracle_lib.bf16_to_f32(bits))]
    ours = oracle_lib.silu(bits)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    theirs = torch.nn.functional.silu(x).view(torch.int16).numpy().view(np.uint16)
    diff = ours != theirs
    assert diff.sum() <= 8, diff.sum()


def test_swiglu_matches_the_torch_composition(oracle_lib):
    """`hidden * silu(gate)` of `y.chunk(2, -1)` in torch bf16 tensor arithmetic (the gated feed-forward module),
    both half orders, against the oracle: bitwise."""
    import torch

    rng = np.random.default_rng(5)
    y = oracle_lib.f32_to_bf16((rng.standard_normal((64, 96)) * 4).astype(np.float32))
    t = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)
    first, second = t.chunk(2, dim=-1)
    for gate_first, (hidden, gate) in ((False, (first, second)), (True, (second, first))):
        theirs = (hidden * torch.nn.functional.silu(gate)).view(torch.int16).numpy().view(np.uint16)
        ours = oracle_lib.swiglu(y, gate_first=gate_first)
        assert ours.shape == (64, 48)
        assert (ours == theirs).all()


def test_silu_closed_forms(oracle_lib):
    """silu(0) = 0, silu(x) = x for large x, -0 far below zero, silu(1) = 1 / (1 + 1/e) = 0.7310585... (bf16
    0.73046875), and swiglu of a zero gate is zero."""
    x = oracle_lib.f32_to_bf16(np.array([0.0, 1.0, 200.0, -200.0], dtype=np.float32))
    s = oracle_lib.bf16_to_f32(oracle_lib.silu(x))
    assert s[0] == 0.0 and s[2] == 200.0 and s[3] == 0.0
    assert s[1] == oracle_lib.bf16_to_f32(oracle_lib.f64_to_bf16(np.array([1.0 / (1.0 + np.exp(-1.0))])))[0]
    y = oracle_lib.f32_to_bf16(np.array([[3.0, -2.0, 0.0, 0.0]], dtype=np.float32))
    assert (oracle_lib.bf16_to_f32(oracle_lib.swiglu(y)) == 0.0).all()


def test_swiglu_planted_mistake_is_caught(oracle_lib):
    """Swapped halves (silu of the hidden half) fail the comparison with torch."""
    import torch

    rng = np.random.default_rng(9)
    y = oracle_lib.f32_to_bf16((rng.standard_normal((32, 64)) * 2).astype(np.float32))
    t = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)
    hidden, gate = t.chunk(2, dim=-1)
    theirs = (hidden * torch.nn.functional.silu(gate)).view(torch.int16).numpy().view(np.uint16)
    assert (oracle_lib.swiglu(y, gate_first=True) != theirs).mean() > 0.5


def test_fp32_sum_bound_holds_for_any_order_and_catches_a_dropped_term(oracle_lib):
    """The device tests' bar for fp32-accumulated low-rank sums (golden_utils.within_fp32_sum_bound): fp32 sums of the
    same products in a random order and in a pairwise tree, each rounded to bf16, are within it of the oracle's
    exactly rounded sums; a sum that drops an outlier channel's product is not."""
    from golden_utils import within_fp32_sum_bound

    m, k, r = 24, 2048, 16
    inp = oracle_lib.make_inputs(m, k, 8, 256, rank=r, outlier_frac=0.01, outlier_scale=30.0, seed=2)
    x = oracle_lib.bf16_to_f32(inp["x"]).astype(np.float32)
    d = oracle_lib.bf16_to_f32(inp["down"]).astype(np.float32)
    ref = oracle_lib.bf16_to_f32(oracle_lib.lowrank_down(inp["x"], inp["down"]))
    prods = x[:, None, :] * d[None, :, :]  # exact in fp32: 8-bit significands
    rng = np.random.default_rng(0)
    shuffled = np.zeros((m, r), np.float32)
    for i in rng.permutation(k):
        shuffled = shuffled + prods[:, :, i]
    tree = prods.copy()
    while tree.shape[-1] > 1:
        tree = tree[..., 0::2] + tree[..., 1::2]
    for sums in (shuffled, tree[..., 0]):
        got = oracle_lib.bf16_to_f32(oracle_lib.f32_to_bf16(sums))
        assert within_fp32_sum_bound(got, ref, x, d)
    outlier = int(np.argmax(np.abs(x).max(axis=0)))
    dropped = prods.sum(axis=2, dtype=np.float32) - prods[:, :, outlier]
    got = oracle_lib.bf16_to_f32(oracle_lib.f32_to_bf16(dropped))
    assert not within_fp32_sum_bound(got, ref, x, d)
