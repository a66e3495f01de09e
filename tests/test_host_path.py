"""The drop-in's host (CPU) path: layers handed host tensors compute on the CPU, as the reference's do
(src/hyperflow_h3_flash/int8.py:161-179, transformer.py:57-58), with the device kernels' definition.

Pinned by the reference's own outputs (the golden fixtures, bit for bit: codes, scales, accumulators, outputs), by
the reference's own CPU test (tests/test_int8.py:51-63, unchanged in substance), by the oracle on random inputs with
outliers for every group, and by closed forms of the rounding helper."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_utils import check_against_composition, fixture_names, load_fixture
from hyperflow_h3_flash_amd import Int8RotLinear, LowRankLinear, host, regular_hadamard
from hyperflow_h3_flash_amd import int8 as int8_mod

FIXTURES = fixture_names()


def bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def make_layer(f, **kw) -> Int8RotLinear:
    layer = Int8RotLinear(f["K"], f["N"], f["G"], **kw)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(f["qweight"]))
        layer.wscale.copy_(torch.from_numpy(f["wscale"]))
    return layer


def reference_quantize(weight: torch.Tensor, group: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The checkpoint format of tests/test_int8.py:31-36: float64 rotation, per-row absmax / 127, rounded codes."""
    blocks = weight.shape[1] // group
    rotated = (weight.double().reshape(-1, blocks, group) @ regular_hadamard(group).double()).reshape(weight.shape)
    wscale = rotated.abs().amax(1) / 127.0
    codes = (rotated / wscale[:, None]).round().clamp(-127, 127).to(torch.int8)
    return codes, wscale.float()


@pytest.mark.parametrize("name", [n for n in FIXTURES if n != "composition"] + ["composition"])
def test_host_layer_is_bitwise_the_reference_golden(name):
    """Codes, scales, accumulators and outputs equal the reference's own `_forward_torch` results."""
    f = load_fixture(name)
    x = bf16_tensor(f["x"])
    xq, sx = host.rotate_quant(x, f["G"])
    np.testing.assert_array_equal(sx.numpy(), f["sx"])
    np.testing.assert_array_equal(xq.numpy(), f["xq"])
    acc = host.int8_gemm_exact(xq, torch.from_numpy(f["qweight"]))
    np.testing.assert_array_equal(acc.numpy().astype(np.int64), f["acc"].astype(np.int64))
    with torch.no_grad():
        y = make_layer(f)(x)
    assert y.dtype == torch.bfloat16 and y.shape == (f["M"], f["N"])
    np.testing.assert_array_equal(bits_of(y), f["y"])


def test_host_fused_extension_against_the_reference_composition(oracle_lib):
    f = load_fixture("composition")
    layer = make_layer(f, rank=f["down"].shape[0], bias=True)
    with torch.no_grad():
        layer.down.weight.copy_(bf16_tensor(f["down"]))
        layer.up.weight.copy_(bf16_tensor(f["up"]))
        layer.bias.copy_(bf16_tensor(f["bias"]))
        y = layer(bf16_tensor(f["x"]))
    # the fused extension's bar against the reference's composition, elementwise
    check_against_composition(bits_of(y), f["y"], f["lowrank"], f["bias"], f["y_composed"])
    # the fused definition (fp32 dequantization, exact low-rank sum and bias, one rounding): bitwise
    u = host.lowrank_down(bf16_tensor(f["x"]), bf16_tensor(f["down"]))
    np.testing.assert_array_equal(bits_of(u), f["u"])  # the reference's bf16 nn.Linear intermediate
    fused = oracle_lib.fused_epilogue(f["acc"], f["sx"], f["wscale"], f["u"], f["up"], f["bias"])
    np.testing.assert_array_equal(bits_of(y), fused)


def test_reference_cpu_test_int8_linear_matches_dense():
    """tests/test_int8.py:51-63 as the reference runs it: fp32 input on the CPU, output in the input's dtype."""
    torch.manual_seed(0)
    weight = torch.randn(96, 128) * 0.05
    x = torch.randn(5, 7, 128)
    layer = Int8RotLinear(128, 96, group=16)
    layer.qweight.copy_(reference_quantize(weight, 16)[0])
    layer.wscale.copy_(reference_quantize(weight, 16)[1])

    y = layer(x)
    reference = x @ weight.T
    assert y.shape == (5, 7, 96) and y.dtype == x.dtype
    error = (y.float() - reference).norm() / reference.norm()
    assert error < 0.02, error


@pytest.mark.parametrize("group", [4, 16, 64, 256, 1024])
def test_host_rotation_matches_the_oracle(oracle_lib, group):
    """Random rows with outlier channels, every power-of-4 group up to 1024 (the host accepts any 4^n)."""
    inp = oracle_lib.make_inputs(37, 2048, 40, group, outlier_frac=0.01, outlier_scale=30.0, seed=group)
    x = bf16_tensor(inp["x"])
    xr = host.round_to_bf16(host.rotate_exact(x, group))
    ref = oracle_lib.rotate(inp["x"], group)
    np.testing.assert_array_equal(bits_of(xr.to(torch.bfloat16)), ref)
    xq, sx = host.rotate_quant(x, group)
    osx, oxq = oracle_lib.quantize(ref)
    np.testing.assert_array_equal(sx.numpy(), osx)
    np.testing.assert_array_equal(xq.numpy(), oxq)
    out = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], group)
    layer = Int8RotLinear(2048, 40, group)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        np.testing.assert_array_equal(bits_of(layer(x)), out["y"])


def test_rounding_helper_rounds_once_to_nearest_even():
    # exact ties at several binades go to the even neighbour; just past a tie goes away from it
    one = 1.0
    ties = torch.tensor([one + 2**-8, one + 3 * 2**-8, -(4.0 + 2**-6), 2.0**-100 * (1 + 2**-8)], dtype=torch.float64)
    np.testing.assert_array_equal(host.round_to_bf16(ties).numpy(),
                                  np.array([1.0, 1.0 + 2**-6, -4.0, 2.0**-100], dtype=np.float32))
    near = torch.tensor([one + 2**-8 + 2**-40, one - 2**-9 - 2**-40], dtype=torch.float64)
    np.testing.assert_array_equal(host.round_to_bf16(near).numpy(),
                                  np.array([1.0 + 2**-7, 1.0 - 2**-8], dtype=np.float32))
    # a value that two roundings (float64 -> fp32 -> bf16) would move: 1 + 2^-8 + 2^-30 rounds up once, but its fp32
    # rounding is the tie 1 + 2^-8, which then rounds down to 1
    v = torch.tensor([one + 2**-8 + 2**-30], dtype=torch.float64)
    assert host.round_to_bf16(v).item() == 1.0 + 2**-7
    assert v.to(torch.float32).to(torch.bfloat16).item() == 1.0
    assert host.round_to_bf16(torch.zeros(3, dtype=torch.float64)).abs().sum().item() == 0.0


def test_host_activations_follow_torch_modules():
    y = (torch.randn(6, 64) * 3).to(torch.bfloat16)
    assert torch.equal(host.activate(y, "gelu_tanh"), torch.nn.functional.gelu(y, approximate="tanh"))
    h, g = y.chunk(2, dim=-1)
    assert torch.equal(host.activate(y, "swiglu"), h * torch.nn.functional.silu(g))
    assert torch.equal(host.activate(y, "swiglu_gate_first"), g * torch.nn.functional.silu(h))
    assert host.activate(y, None) is y


def test_kernels_is_none_without_the_library(monkeypatch):
    """The reference's `_kernels()` returns None when its kernels are unavailable (int8.py:184-187); the host path
    still runs, while a device tensor would raise (there is no device fallback)."""
    from hyperflow_h3_flash_amd import _native

    def missing():
        raise RuntimeError("missing")

    monkeypatch.setattr(_native, "library", missing)
    int8_mod._kernels.cache_clear()
    try:
        assert int8_mod._kernels() is None
        layer = Int8RotLinear(64, 32, group=16)
        assert layer(torch.randn(3, 64)).shape == (3, 32)
    finally:
        int8_mod._kernels.cache_clear()


def test_host_forward_clears_the_shared_input():
    to_q = Int8RotLinear(64, 32, group=16)
    to_q.keep_input = True
    Int8RotLinear._last_input.update(x=object(), version=0, group=16, value=None)
    to_q(torch.randn(2, 64))
    assert not Int8RotLinear._last_input


def test_lowrank_linear_on_the_host_is_the_reference_composition():
    """LowRankLinear on host tensors and in float32/float64 modules is ``up(down(x))`` in the module's dtype: the
    re-padding identity of tests/test_transformer.py:96-115 holds to 1e-12 in float64."""
    torch.manual_seed(3)
    layer = LowRankLinear(64, 48, 16).double()
    with torch.no_grad():
        layer.down.weight[5:] = 0
        layer.up.weight[:, 5:] = 0
    x = torch.randn(4, 7, 64, dtype=torch.float64)
    expected = layer.up(layer.down(x))
    torch.testing.assert_close(layer(x), expected, rtol=0, atol=0)
    assert layer.pad_rank() and layer.rank == 64
    torch.testing.assert_close(layer(x), expected, rtol=1e-12, atol=1e-12)
    bf = LowRankLinear(64, 48, 16).to(torch.bfloat16)
    xb = torch.randn(3, 64).to(torch.bfloat16)
    assert torch.equal(bf(xb), bf.up(bf.down(xb)))
