"""The config seam and checkpoint format (src/hyperflow_h3_flash/transformer.py:112-122,194-203,
tests/test_transformer.py:25-39,136-146,164-175, tests/test_int8.py:31-36), on a toy module tree. CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from hyperflow_h3_flash_amd import Int8RotLinear
from hyperflow_h3_flash_amd.convert import apply_quantization, quantize_weight, replace_linear


class Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.to_q = nn.Linear(d, d, bias=False)
        self.to_k = nn.Linear(d, d, bias=False)
        self.to_v = nn.Linear(d, d, bias=False)
        self.to_out = nn.ModuleList([nn.Linear(d, d, bias=False), nn.Dropout(0.0)])


class Block(nn.Module):
    def __init__(self, d, ffn):
        super().__init__()
        self.attn = Attn(d)
        self.ff = nn.Module()
        self.ff.net = nn.ModuleList([nn.Linear(d, ffn, bias=False), nn.GELU(), nn.Linear(ffn, d, bias=False)])


class Toy(nn.Module):
    def __init__(self, d=64, ffn=128, blocks=3):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([Block(d, ffn) for _ in range(blocks)])
        self.proj = nn.Linear(d, d)  # has a bias


QUANT = {
    "method": "int8_convrot",
    "group": 16,
    "linears": ["transformer_blocks.2.attn.to_k", "transformer_blocks.2.ff.net.2",
                "transformer_blocks.1.attn.to_q", "transformer_blocks.1.attn.to_v",
                "transformer_blocks.1.attn.to_out.0"],
}


def test_quantization_config_replaces_the_named_linears():
    model = Toy()
    names = apply_quantization(model, QUANT)
    assert names == QUANT["linears"]
    assert isinstance(model.transformer_blocks[2].attn.to_k, Int8RotLinear)
    assert isinstance(model.transformer_blocks[2].ff.net[2], Int8RotLinear)
    assert isinstance(model.transformer_blocks[1].attn.to_out[0], Int8RotLinear)
    assert model.transformer_blocks[2].ff.net[2].in_features == 128
    assert isinstance(model.transformer_blocks[0].attn.to_q, nn.Linear)
    assert model.transformer_blocks[2].attn.to_k.group == 16


def test_q_and_k_keep_their_input_v_does_not():
    model = Toy()
    apply_quantization(model, QUANT)
    attn = model.transformer_blocks[1].attn
    assert (attn.to_q.keep_input, attn.to_v.keep_input) == (True, False)
    assert model.transformer_blocks[2].attn.to_k.keep_input is True
    assert model.transformer_blocks[2].ff.net[2].keep_input is False


def test_unknown_quantization_method_is_rejected():
    with pytest.raises(ValueError, match="unsupported quantization method"):
        apply_quantization(Toy(), {"method": "nf4", "group": 16, "linears": []})
    assert apply_quantization(Toy(), None) == []


def test_only_bias_free_linears_are_replaced():
    model = Toy()
    with pytest.raises(TypeError, match="bias-free"):
        replace_linear(model, "proj", Int8RotLinear, 16)
    with pytest.raises(TypeError):
        replace_linear(model, "transformer_blocks.0.ff.net.1", Int8RotLinear, 16)


def test_quantized_state_keeps_int8_and_fp32_under_a_bf16_cast():
    model = Toy()
    apply_quantization(model, QUANT)
    model = model.to(torch.bfloat16)
    layer = model.transformer_blocks[2].attn.to_k
    assert layer.qweight.dtype == torch.int8
    # nn.Module.to(dtype) converts floating parameters; the reference keeps wscale fp32 through diffusers'
    # _keep_in_fp32_modules at load time (transformer.py:129-133). Restoring it is the loader's job:
    assert layer.wscale.dtype == torch.bfloat16
    layer.wscale.data = layer.wscale.data.float()
    assert set(layer.state_dict()) == {"qweight", "wscale"}


def test_quantize_weight_matches_the_oracle_restatement(oracle_lib):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((40, 256)) * 0.02
    q, ws = quantize_weight(torch.from_numpy(w), 64)
    q_ref, ws_ref = oracle_lib.quantize_weight(w, 64)
    np.testing.assert_array_equal(q.numpy(), q_ref)
    np.testing.assert_allclose(ws.numpy(), ws_ref, rtol=1e-7)
    with pytest.raises(ValueError):
        quantize_weight(torch.zeros(4, 100), 16)


def test_dequantized_weight_reconstructs_the_dense_one(oracle_lib):
    torch.manual_seed(0)
    w = torch.randn(96, 128) * 0.05
    q, ws = quantize_weight(w, 16)
    h = torch.block_diag(*[torch.from_numpy(oracle_lib.regular_hadamard(16))] * 8).double()
    back = (q.double() * ws.double()[:, None]) @ h.T
    assert ((back - w.double()).norm() / w.double().norm()) < 0.01
