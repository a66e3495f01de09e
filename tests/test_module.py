"""The drop-in module's host-side behaviour, mirroring the reference's CPU tests (tests/test_int8.py:39-90,
176-185; tests/test_transformer.py:164-175). CPU only: no kernel runs here."""

from __future__ import annotations

import io
from types import SimpleNamespace

import pytest
import torch
from safetensors.torch import load, save

from hyperflow_h3_flash_amd import (
    KERNEL_OPTIONS,
    Int8RotLinear,
    hadamard_factors,
    regular_hadamard,
    resolve_int8_gemm,
    set_kernel_options,
)
from hyperflow_h3_flash_amd import int8 as int8_mod


@pytest.mark.parametrize("group", [4, 16, 64, 256])
def test_regular_hadamard_is_orthonormal_and_symmetric(group):
    h = regular_hadamard(group).double()
    torch.testing.assert_close(h @ h.T, torch.eye(group, dtype=torch.float64))
    torch.testing.assert_close(h, h.T)
    assert h.dtype == torch.float64 and regular_hadamard(group).dtype == torch.float32


def test_regular_hadamard_rejects_non_powers_of_four():
    with pytest.raises(ValueError):
        regular_hadamard(32)


@pytest.mark.parametrize("group", [256, 1024, 4096])
def test_hadamard_factors_rebuild_the_rotation(group):
    ga, gb = hadamard_factors(group)
    assert ga >= 16 and gb >= 16
    torch.testing.assert_close(torch.kron(regular_hadamard(ga), regular_hadamard(gb)), regular_hadamard(group))


def test_small_groups_have_no_factors():
    assert hadamard_factors(16) is None and hadamard_factors(64) is None


def test_int8_linear_state_is_two_frozen_parameters():
    layer = Int8RotLinear(64, 32, group=16)
    assert set(layer.state_dict()) == {"qweight", "wscale"}
    assert not list(layer.buffers())
    assert not any(p.requires_grad for p in layer.parameters())
    assert layer.qweight.dtype == torch.int8 and layer.qweight.shape == (32, 64)
    assert layer.wscale.dtype == torch.float32 and layer.wscale.shape == (32,)
    assert layer.keep_input is False
    assert repr(layer) == "Int8RotLinear(in_features=64, out_features=32, group=16)"


def test_in_features_must_be_a_multiple_of_the_group():
    with pytest.raises(ValueError, match="multiple of the Hadamard group"):
        Int8RotLinear(100, 32, group=16)


def test_extension_tensors_follow_lowrank_layout():
    layer = Int8RotLinear(64, 32, group=16, rank=8, bias=True)
    sd = layer.state_dict()
    assert set(sd) == {"qweight", "wscale", "down.weight", "up.weight", "bias"}
    assert sd["down.weight"].shape == (8, 64) and sd["up.weight"].shape == (32, 8)
    assert all(sd[k].dtype == torch.bfloat16 for k in ("down.weight", "up.weight", "bias"))
    assert not any(p.requires_grad for p in layer.parameters())
    assert "rank=8" in repr(layer) and "bias=True" in repr(layer)


def test_activation_option_adds_no_state_and_is_checked():
    plain = Int8RotLinear(64, 32, group=16, rank=8)
    fused = Int8RotLinear(64, 32, group=16, rank=8, activation="gelu_tanh")
    assert fused.state_dict().keys() == plain.state_dict().keys()
    assert plain.activation is None and "activation" not in repr(plain)
    assert "activation=gelu_tanh" in repr(fused)
    with pytest.raises(ValueError, match="unsupported activation"):
        Int8RotLinear(64, 32, group=16, activation="relu")


def test_state_dict_round_trip_keeps_storage_dtypes():
    layer = Int8RotLinear(64, 32, group=16)
    with torch.no_grad():
        layer.qweight.copy_(torch.randint(-127, 128, (32, 64), dtype=torch.int8))
        layer.wscale.copy_(torch.rand(32))
    blob = save(layer.state_dict())
    again = Int8RotLinear(64, 32, group=16)
    again.load_state_dict(load(blob))
    assert again.qweight.dtype == torch.int8 and again.wscale.dtype == torch.float32
    assert torch.equal(again.qweight, layer.qweight) and torch.equal(again.wscale, layer.wscale)
    # a bf16 model cast must keep the scale in fp32 only if asked to; plain .to(bf16) converts floating params
    buf = io.BytesIO()
    torch.save(layer.state_dict(), buf)
    buf.seek(0)
    assert set(torch.load(buf, weights_only=True)) == {"qweight", "wscale"}


def test_kernel_options_are_checked_and_default_to_the_release_arithmetic():
    assert KERNEL_OPTIONS == {"int8_gemm": "auto", "rotate_quant": "dense"}
    with pytest.raises(ValueError, match="int8_gemm"):
        set_kernel_options(int8_gemm="cutlass")
    with pytest.raises(ValueError, match="rotate_quant"):
        set_kernel_options(rotate_quant="fast")
    saved = dict(KERNEL_OPTIONS)
    try:
        for choice in ("auto", "triton", "cublas", "sgl", "bf16"):
            set_kernel_options(int8_gemm=choice)
            assert resolve_int8_gemm(torch.device("cpu")) == int8_mod.BACKEND
    finally:
        KERNEL_OPTIONS.update(saved)


def test_arithmetic_options_are_checked_and_default_to_the_torch_path():
    from hyperflow_h3_flash_amd import ARITHMETIC_OPTIONS, ROTATE_ARITHMETICS, set_arithmetic_options

    assert ARITHMETIC_OPTIONS == {"rotate_quant": "bf16_div"}
    assert ROTATE_ARITHMETICS == {"bf16_div": 0, "f32_recip": 1}  # the C ABI's HF_ROTATE_* codes
    with pytest.raises(ValueError, match="arithmetic"):
        set_arithmetic_options(rotate_quant="dense")
    try:
        set_arithmetic_options(rotate_quant="f32_recip")
        assert ARITHMETIC_OPTIONS["rotate_quant"] == "f32_recip"
    finally:
        set_arithmetic_options(rotate_quant="bf16_div")


def test_shared_quantization_is_not_reused_across_arithmetics():
    from hyperflow_h3_flash_amd import set_arithmetic_options

    calls = []
    kernels = SimpleNamespace(rotate_quant=lambda x2, group: calls.append(1) or (x2, group))
    to_q, to_k = Int8RotLinear(16, 16, group=16), Int8RotLinear(16, 16, group=16)
    to_q.keep_input = True
    x = torch.randn(4, 16)
    to_q._quantize(x, x, kernels)
    try:
        set_arithmetic_options(rotate_quant="f32_recip")
        to_k._quantize(x, x, kernels)
    finally:
        set_arithmetic_options(rotate_quant="bf16_div")
    assert len(calls) == 2 and not Int8RotLinear._last_input


def test_shared_quantization_works_under_inference_mode():
    calls = []
    kernels = SimpleNamespace(rotate_quant=lambda x2, group: calls.append(1) or (x2, group))
    to_q, to_k = Int8RotLinear(16, 16, group=16), Int8RotLinear(16, 16, group=16)
    to_q.keep_input = True
    with torch.inference_mode():
        x = torch.randn(4, 16)
        to_q._quantize(x, x, kernels)
        to_k._quantize(x, x, kernels)
    assert len(calls) == 1 and not Int8RotLinear._last_input


def test_shared_quantization_invalidated_by_in_place_change_and_other_tensors():
    calls = []
    kernels = SimpleNamespace(rotate_quant=lambda x2, group: calls.append(1) or (x2, group))
    to_q, to_k = Int8RotLinear(16, 16, group=16), Int8RotLinear(16, 16, group=16)
    to_q.keep_input = to_k.keep_input = True
    x = torch.randn(4, 16)
    to_q._quantize(x, x, kernels)
    to_k._quantize(x, x, kernels)
    assert len(calls) == 1
    x.mul_(2)  # bumps the version counter
    to_k._quantize(x, x, kernels)
    assert len(calls) == 2
    to_k._quantize(x.clone(), x, kernels)
    assert len(calls) == 3
    to_other = Int8RotLinear(64, 16, group=64)
    to_other._quantize(x, x, kernels)  # same tensor, other group
    assert len(calls) == 4
    Int8RotLinear._last_input.clear()


def test_device_groups_are_checked():
    with pytest.raises(ValueError, match="power of 4"):
        int8_mod._check_group(128)
    with pytest.raises(ValueError, match="not supported"):
        int8_mod._check_group(65536)
    for g in (4, 16, 64, 256, 1024, 4096, 16384):
        int8_mod._check_group(g)
