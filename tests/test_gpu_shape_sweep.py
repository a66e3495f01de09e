"""Shapes on both sides of every boundary between the GEMM's dispatch paths, against the oracle.

The library picks, by M, N and the device's CU count C: the single-pass few-row GEMM (M <= 64 and between C / 4 and C
slices of 32 weight rows), the split few-row GEMM with its finishing pass, the 256 x 128 tiles of the mid-size GEMM,
and the persistent 256 x 256 tiles (whole or split over K). The shapes below sit at those thresholds (computed from
the device's C), with ragged N and M and K values that end inside a 128-byte stage, and shapes on either side of
the measured cost models' choices (whole tiles against a K split, a second round of mid-size tiles). Bars: without
a low-rank branch and bias, codes, scales and outputs bitwise the oracle's; with a rank-32 branch and a bias, every
output within one bf16 ulp of the oracle's fused definition on the device's own low-rank intermediate (the bars of
the other GEMM tests).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from test_gpu_skinny_fused import bits_of, layer_operands

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def _cus() -> int:
    return torch.cuda.get_device_properties(0).multi_processor_count if torch.cuda.is_available() else 256


def _shapes():
    c = _cus()
    lo, hi = 32 * ((c + 3) // 4), 32 * c  # widths of C / 4 and C slices of 32 weight rows
    return [
        # single pass against split at M <= 64
        (64, 1040, lo, 0), (64, 1040, lo - 32, 0), (64, 1040, hi, 0), (64, 1040, hi + 16, 0), (1, 2064, lo, 0),
        (65, 1040, lo + 48, 0), (33, 2064, hi - 16, 32),
        # few rows, split, and the mid-size tiles
        (129, 1040, 4096, 0), (200, 2064, hi + 16, 32), (257, 1040, 4112, 0), (512, 1040, 4096, 32),
        (1000, 1040, 2064, 0),
        # persistent 256 x 256 tiles: one round exactly, one tile more, ragged edges
        (4096, 256, 4096, 0), (4100, 256, 4112, 32), (2048, 256, 8192, 0),
        # fewer 256 x 256 tiles than CUs where whole tiles beat a K split, and where a second round of mid-size
        # tiles loses to them
        (2048, 1024, 5120, 0), (640, 1024, 15360, 32),
    ]


@pytest.mark.parametrize("shape", _shapes(), ids=lambda s: "m{}_k{}_n{}_r{}".format(*s))
def test_dispatch_boundaries_match_oracle(oracle_lib, shape):
    from hyperflow_h3_flash_amd.int8 import int8_matmul

    m, k, n, rank = shape
    bias = rank > 0
    inp, g, q, sx, w, ws, kw = layer_operands(oracle_lib, m, k, n, rank, bias, seed=m * 7 + n + k)
    print(f"dispatch boundary M={m} K={k} N={n} rank={rank} bias={bias}", flush=True)
    y = int8_matmul(q, w, sx, ws, **kw)
    torch.cuda.synchronize()
    ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), ref["sx"].view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), ref["xq"])
    if not rank:
        np.testing.assert_array_equal(bits_of(y), ref["y"])
        return
    fused = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(ref["acc"], ref["sx"], inp["wscale"], bits_of(kw["u"]),
                                                             inp["up"], inp["bias"]))
    got = oracle_lib.bf16_to_f32(bits_of(y))
    assert (np.abs(got - fused) <= np.abs(fused) * 2.0**-7 + 1e-6).all()
    assert (got == fused).mean() > 0.98
