"""Hadamard groups of 1024 and more on the device, against the oracle: the reference accepts any power of 4
(int8.py:100-109), the release uses 256. A 1024 group is one 1024-element tile and runs on the tile kernels (one more
radix-4 stage after a second transpose through LDS: the row, register, and row-buffer layouts); 4096 and 16384 run
on rotate_quant_wide_kernel (one workgroup per row, the row's fp64 sums in LDS).

Bar: codes and scales bitwise the oracle's under both arithmetics (the torch path's bf16 value with a true division;
the reference's CUDA kernels' fp32 value with a reciprocal multiply), and the layer output bitwise the oracle's
(r = 0, no bias) or within one bf16 ulp of the fused definition and 1e-2 of the composition (low-rank term and bias).
Rows with outlier channels, ragged row counts, a row stride wider than K, rows up to 24576 elements, and the refusal
of rows too long for the fp64 LDS row (groups of 4096 and more).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


CASES = [
    # group, m, k
    (1024, 1, 1024),       # one workgroup per row
    (1024, 67, 5120),
    (1024, 2000, 5120),    # rows held in registers, one wave per row
    (1024, 1500, 14336),   # rows held in registers, three waves per row
    (1024, 3, 19456),
    (1024, 5, 24576),      # one wave per row with an LDS row buffer
    (4096, 20, 8192),      # one workgroup per row, fp64 row in LDS
    (4096, 9, 16384),
    (16384, 3, 16384),
]


def sample_rows(m, seed, count=24):
    if m <= count:
        return np.arange(m)
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([rng.choice(m, size=count, replace=False), [0, m - 1]]))


@pytest.mark.parametrize("group,m,k", CASES)
def test_wide_group_rotation_matches_the_oracle(oracle_lib, group, m, k):
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    inp = oracle_lib.make_inputs(m, k, 8, group, outlier_frac=0.005, outlier_scale=30.0, seed=group + m + k)
    q, s = rotate_quant(to_dev_bf16(inp["x"]), group)
    rows = sample_rows(m, m + k)
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(inp["x"][rows], group))
    np.testing.assert_array_equal(s.cpu().numpy()[rows], sx)
    np.testing.assert_array_equal(q.cpu().numpy()[rows], xq)
    assert bool(torch.isfinite(s).all()) and bool((s > 0).all())


@pytest.mark.parametrize("group,m,k", [(1024, 67, 5120), (1024, 9, 24576), (4096, 9, 16384), (16384, 3, 16384)])
def test_wide_group_f32_recip_matches_the_oracle(oracle_lib, group, m, k):
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    inp = oracle_lib.make_inputs(m, k, 8, group, outlier_frac=0.01, outlier_scale=30.0, seed=3 * group + m)
    q, s = rotate_quant(to_dev_bf16(inp["x"]), group, arithmetic="f32_recip")
    sx, xq = oracle_lib.quantize_recip(oracle_lib.rotate_f32(inp["x"], group))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)


def test_wide_group_zero_rows_wide_spans_and_strides(oracle_lib):
    """Zero rows, values spanning many binades, and x a column slice of a wider tensor."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    rng = np.random.default_rng(11)
    m, k, g = 24, 4096, 1024
    x = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-20, 12, size=(m, k)))).astype(np.float32)
    x[5] = 0.0
    x[9, ::3] = 0.0
    bits = oracle_lib.f32_to_bf16(x)
    wide = torch.zeros(m, k + 512, device=DEV, dtype=torch.bfloat16)
    wide[:, :k] = to_dev_bf16(bits)
    q, s = rotate_quant(wide[:, :k], g)
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(bits, g))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)
    assert s[5].item() == np.float32(1e-12) / np.float32(127.0) and not q[5].any()


def test_wide_group_rows_too_long_for_the_lds_row_are_refused():
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    x = torch.zeros(2, 20480, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="size"):
        rotate_quant(x, 4096)
    for g in (256, 1024):  # the same rows with a 256 or 1024 group take the tile kernels
        q, _ = rotate_quant(x, g)
        assert not q.any()


@pytest.mark.parametrize("m,k,n,g,r,bias", [(40, 5120, 384, 1024, 0, False), (40, 5120, 384, 1024, 16, True),
                                           (700, 7168, 1024, 1024, 32, False), (300, 8192, 512, 4096, 0, False),
                                           (300, 8192, 512, 4096, 16, True)])
def test_layer_with_a_wide_group(oracle_lib, m, k, n, g, r, bias):
    """The whole layer (one library call: the rotation, then the low-rank down projection in its own launch, the
    GEMM) against the oracle."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    inp = oracle_lib.make_inputs(m, k, n, g, rank=r, bias=bias, outlier_frac=0.005, outlier_scale=30.0, seed=m + g)
    layer = Int8RotLinear(k, n, g, rank=r, bias=bias).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        if r:
            layer.down.weight.copy_(to_dev_bf16(inp["down"]))
            layer.up.weight.copy_(to_dev_bf16(inp["up"]))
        if bias:
            layer.bias.copy_(to_dev_bf16(inp["bias"]))
        y = layer(to_dev_bf16(inp["x"]))
    torch.cuda.synchronize()
    ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    got = bits_of(y)
    if not r and not bias:
        np.testing.assert_array_equal(got, ref["y"])
        return
    u_ref = oracle_lib.lowrank_down(inp["x"], inp["down"]) if r else None
    fused = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(ref["acc"], ref["sx"], inp["wscale"], u_ref,
                                                             inp.get("up") if r else None,
                                                             inp.get("bias") if bias else None))
    g32 = oracle_lib.bf16_to_f32(got)
    assert (np.abs(g32 - fused) <= np.abs(fused) * 2.0**-7 + 1e-6).all()
    comp = oracle_lib.bf16_to_f32(oracle_lib.composition(ref["y"], inp["x"], inp.get("down") if r else None,
                                                         inp.get("up") if r else None,
                                                         inp.get("bias") if bias else None))
    assert np.abs(g32 - comp).max() / np.abs(comp).max() <= 1e-2
