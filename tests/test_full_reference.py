"""The reference's own CPU path at four benchmark sizes against the oracle (CPU).

The fixtures (tests/golden/full/*.npz) hold the reference ``Int8RotLinear.forward`` on CPU tensors at M=1024,
K=N=3072 (a single layer of 1024 tokens), M=32768, K=5120, N=15360 (the headline QKV projection), M=32768, K=13824, N=5120
(the FFN down projection) and M=41344, K=5120, N=15360 (a 41344-token block at the QKV width), as digests plus every
position where it differs from the exact-sum definition. These tests check what the fixtures claim about those
differences, and that the oracle reproduces the reference everywhere else on the rows it can afford to recompute:

* every listed rotated value is the exact sum's rounding on the oracle's side and within the fp32 accumulation
  error bound of the exact sum on the reference's (`golden_utils.classify_rotation_mismatches`), and every listed
  code moves by one;
* no scale differs, and every output that differs lies in a row whose codes differ;
* M=1024, K=N=3072: the oracle's codes and scales of all 1024 rows give the reference's digest after the listed positions
  are set; the larger ones: the oracle's codes and outputs of the moved rows match the listed values, and its outputs
  of the sampled rows are the reference's.

The device is checked against the same digests in test_gpu_full_reference.py.
"""

from __future__ import annotations

import hashlib

import numpy as np
import pytest

from full_reference import FULL_FIXTURES, LARGE_FIXTURES, inputs, load, patched_digest
from golden_utils import classify_rotation_mismatches


def check_rotation_differences(fx: dict, x_bits: np.ndarray, x_row_ids: np.ndarray, oracle_lib) -> None:
    """Every listed rotated-value difference is explained by the reference's fp32 accumulation. `x_bits` holds the
    rows `x_row_ids` (sorted) of x, among them every row with a listed difference."""
    k, g = int(fx["shape"][1]), int(fx["shape"][3])
    rows = np.unique(fx["xr_idx"] // k)
    x_rows = x_bits[np.searchsorted(x_row_ids, rows)]
    exact = oracle_lib.rotate(x_rows, g)
    other = exact.copy()
    pos = {int(r): i for i, r in enumerate(rows)}
    for flat, ref_v, orc_v in zip(fx["xr_idx"], fx["xr_ref"], fx["xr_oracle"]):
        assert exact[pos[int(flat // k)], int(flat % k)] == orc_v
        other[pos[int(flat // k)], int(flat % k)] = ref_v
    count, unexplained = classify_rotation_mismatches(x_rows, exact, other, g, limit=10**6)
    assert count == fx["xr_idx"].size and not unexplained, unexplained[:5]


@pytest.mark.parametrize("name", FULL_FIXTURES)
def test_listed_differences_are_single_steps(name):
    fx = load(name)
    m, k, n, _ = (int(v) for v in fx["shape"])
    assert fx["sx_idx"].size == 0, "no per-token scale differs"
    # Rotated values: adjacent bf16 values (same sign, bit patterns one apart).
    r, o = fx["xr_ref"].astype(np.int32), fx["xr_oracle"].astype(np.int32)
    assert np.all(r != o) and np.all((r >> 15) == (o >> 15))
    # Codes: one step apart, and each moved code sits on a rotated value that moved.
    assert np.all(np.abs(fx["xq_ref"].astype(np.int32) - fx["xq_oracle"].astype(np.int32)) == 1)
    assert np.isin(fx["xq_idx"], fx["xr_idx"]).all()
    # Outputs: only in rows whose codes moved.
    assert np.isin(fx["y_idx"] // n, fx["xq_idx"] // k).all()
    assert fx["y_idx"].max(initial=-1) < m * n


def test_m1024_codes_and_scales_all_rows(oracle_lib):
    fx = load("full_cfg1")
    inp = inputs(fx)
    g = int(fx["shape"][3])
    xr = oracle_lib.rotate(inp["x"], g)
    sx, xq = oracle_lib.quantize(xr)
    check_rotation_differences(fx, inp["x"], np.arange(inp["x"].shape[0]), oracle_lib)
    assert np.array_equal(sx.view(np.uint32), fx["sx"].view(np.uint32))
    assert patched_digest(xq, fx["xq_idx"], fx["xq_ref"]) == str(fx["xq_sha256"])
    rows = fx["sample_rows"]
    y = oracle_lib.epilogue(oracle_lib.int8_gemm(xq[rows], inp["qweight"]), sx[rows], inp["wscale"])
    assert np.array_equal(y, fx["y_sample"])


@pytest.mark.parametrize("name", LARGE_FIXTURES)
def test_moved_and_sampled_rows(oracle_lib, name):
    fx = load(name)
    m, k, n, g = (int(v) for v in fx["shape"])
    moved = np.unique(fx["xq_idx"] // k)
    rows = np.union1d(moved, fx["sample_rows"])
    need = np.union1d(rows, np.unique(fx["xr_idx"] // k))  # only these rows of x are kept
    inp = inputs(fx, x_rows=need)
    check_rotation_differences(fx, inp["x"], need, oracle_lib)
    xr = oracle_lib.rotate(inp["x"][np.searchsorted(need, rows)], g)
    sx, xq = oracle_lib.quantize(xr)
    assert np.array_equal(sx.view(np.uint32), fx["sx"][rows].view(np.uint32))
    # The listed code differences are exactly where the oracle's codes of the moved rows differ from the listed
    # reference values.
    pos = {int(r): i for i, r in enumerate(rows)}
    for flat, ref_v, orc_v in zip(fx["xq_idx"], fx["xq_ref"], fx["xq_oracle"]):
        assert xq[pos[int(flat // k)], int(flat % k)] == orc_v != ref_v
    y = oracle_lib.epilogue(oracle_lib.int8_gemm(xq, inp["qweight"]), sx, inp["wscale"])
    for flat, orc_v in zip(fx["y_idx"], fx["y_oracle"]):
        assert y[pos[int(flat // n)], int(flat % n)] == orc_v
    samples = [int(np.searchsorted(rows, r)) for r in fx["sample_rows"]]
    assert np.array_equal(y[samples], fx["y_sample"])
    assert np.unique(fx["y_idx"]).size == fx["y_idx"].size
