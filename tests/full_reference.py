"""Shared helpers of the full-size reference fixtures (tests/golden/full/*.npz, written by make_golden_full.py).

A fixture holds the reference CPU path's output at a benchmark size as digests plus the list of positions where it
differs from the exact-sum definition. `patched_digest` sets those positions of an array to the reference's values
and hashes it: for an array equal to the definition everywhere the result is the reference's digest.
"""

from __future__ import annotations

import hashlib
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "full")
FULL_FIXTURES = ("full_cfg1", "full_cfg2", "full_cfg3_down", "full_cfg4_qkv")
#: the fixtures whose outputs the oracle recomputes on the moved and sampled rows only (too large for every row)
LARGE_FIXTURES = FULL_FIXTURES[1:]


def load(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {key: z[key] for key in z.files}


def inputs(fx: dict, x_rows=None) -> dict:
    """The fixture's inputs, rebuilt from its seed; with `x_rows` (sorted) only those rows of x."""
    from oracle import oracle as O

    m, k, n, g = (int(v) for v in fx["shape"])
    return O.make_inputs(m, k, n, g, outlier_frac=float(fx["outlier_frac"]),
                         outlier_scale=float(fx["outlier_scale"]), seed=int(fx["seed"]), x_rows=x_rows)


def patched_digest(a: np.ndarray, idx: np.ndarray, ref_values: np.ndarray) -> str:
    flat = np.ascontiguousarray(a).reshape(-1).copy()
    flat[idx] = ref_values
    return hashlib.sha256(flat.tobytes()).hexdigest()
