"""The feed-forward activation fused into the INT8 GEMM epilogue (tanh-GELU on the bf16 linear output).

Bars: the fused output is the oracle's tanh-GELU (torch's formula in fp32, pinned against torch in test_oracle.py)
of the same layer's unfused output: within 1e-3 of the output's maximum everywhere, and bitwise on at least 99.9 %
of the elements whose input is >= -3. Below -3 the formula's `1 + tanh(u)` cancels (tanh is within 1e-4 of -1), so
the last fp32 bits of tanh, which differ between any two implementations (the device uses exp2 and a reciprocal,
torch its own tanh), decide the bf16 rounding of values below 1e-2 in magnitude. With the low-rank branch and a
bias: within 1e-2 (max |y - y_ref| / max |y_ref|) of the reference's module composition followed by the
activation. Every GEMM path is covered: 256 x 256 tiles, few-row split K and the skinny kernel.
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


def check_gelu(got_bits, pre_bits, lib):
    """`got_bits` against the oracle's activation of the pre-activation bf16 values `pre_bits`."""
    ref_bits = lib.gelu_tanh(pre_bits)
    got, ref = lib.bf16_to_f32(got_bits), lib.bf16_to_f32(ref_bits)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    well_conditioned = lib.bf16_to_f32(pre_bits) >= -3.0
    exact = (got_bits == ref_bits)[well_conditioned].mean()
    assert rel <= 1e-3, (rel, exact)
    assert exact >= 0.999, (rel, exact)


# (M, K, N): 256 x 256 tiles with a ragged edge, few rows (split K), at most 64 rows (skinny kernel)
SHAPES = [(600, 1024, 700), (200, 2048, 512), (40, 1024, 300), (1, 512, 64)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("rank,bias", [(0, False), (64, True), (32, False)])
def test_gelu_epilogue_is_gelu_of_the_linear_output(oracle_lib, m, k, n, rank, bias):
    from hyperflow_h3_flash_amd.int8 import int8_matmul, lowrank_down, rotate_quant

    inp = oracle_lib.make_inputs(m, k, n, 256, rank=rank, bias=bias, outlier_frac=0.01, outlier_scale=20.0,
                                 seed=m + k + n + rank)
    x = to_dev_bf16(inp["x"])
    w = torch.from_numpy(inp["qweight"]).to(DEV)
    ws = torch.from_numpy(inp["wscale"]).to(DEV)
    q, sx = rotate_quant(x, 256)
    kw = {}
    if rank:
        kw = dict(u=lowrank_down(x, to_dev_bf16(inp["down"])), up=to_dev_bf16(inp["up"]))
    if bias:
        kw["bias"] = to_dev_bf16(inp["bias"])
    plain = int8_matmul(q, w, sx, ws, **kw)
    fused = int8_matmul(q, w, sx, ws, activation="gelu_tanh", **kw)
    torch.cuda.synchronize()
    check_gelu(bits_of(fused), bits_of(plain), oracle_lib)


def test_gelu_layer_against_the_reference_composition(oracle_lib):
    """Int8RotLinear(activation="gelu_tanh") with the low-rank branch and a bias against gelu(Int8RotLinear(x) +
    LowRankLinear(x) + bias), the reference modules composed in bf16."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    m, k, n, g, r = 300, 1024, 520, 256, 64
    inp = oracle_lib.make_inputs(m, k, n, g, rank=r, bias=True, outlier_frac=0.005, outlier_scale=30.0, seed=7)
    layer = Int8RotLinear(k, n, g, rank=r, bias=True, activation="gelu_tanh").to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        layer.down.weight.copy_(to_dev_bf16(inp["down"]))
        layer.up.weight.copy_(to_dev_bf16(inp["up"]))
        layer.bias.copy_(to_dev_bf16(inp["bias"]))
        y = layer(to_dev_bf16(inp["x"]))
    out = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    comp = oracle_lib.composition(out["y"], inp["x"], inp["down"], inp["up"], inp["bias"])
    ref = oracle_lib.bf16_to_f32(oracle_lib.gelu_tanh(comp))
    got = oracle_lib.bf16_to_f32(bits_of(y))
    tolerance = 1e-2  # max |y - y_ref| / max |y_ref| against the reference's bf16 composition + activation
    assert np.abs(got - ref).max() / np.abs(ref).max() <= tolerance


def test_gelu_layer_without_extension_is_gelu_of_the_reference_output(oracle_lib):
    """No low-rank branch, no bias: the activation of the reference's bitwise output."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    m, k, n, g = 257, 512, 300, 64
    inp = oracle_lib.make_inputs(m, k, n, g, seed=11)
    layer = Int8RotLinear(k, n, g, activation="gelu_tanh").to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        y = layer(to_dev_bf16(inp["x"]))
    check_gelu(bits_of(y), oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)["y"], oracle_lib)
