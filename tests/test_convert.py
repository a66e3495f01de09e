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


# ------------------------------------------------------------------------------------------ checkpoint partitions

RANKS = {"transformer_blocks.0.attn.to_q": 8, "transformer_blocks.0.attn.to_out.0": 16}


def partition_config():
    return {"lowrank_ranks": dict(RANKS), "quantization": dict(QUANT), "dropped_blocks": []}


def filled_model(seed=0):
    from hyperflow_h3_flash_amd.convert import load_quantized, prepare_model

    torch.manual_seed(seed)
    model = prepare_model(Toy(), partition_config())
    for module in model.modules():
        if isinstance(module, Int8RotLinear):
            load_quantized(module, torch.randn(module.out_features, module.in_features) * 0.02)
    return model


def test_save_and_load_keep_the_storage_dtypes(tmp_path):
    """tests/test_transformer.py:164-175: qweight int8 and wscale fp32 under a bf16 model; low-rank factors bf16."""
    from hyperflow_h3_flash_amd import LowRankLinear
    from hyperflow_h3_flash_amd.convert import load_partition, save_partition

    model = filled_model()
    save_partition(model, str(tmp_path), partition_config())
    fresh = Toy().to(torch.bfloat16)
    missing, unexpected = load_partition(fresh, str(tmp_path))
    assert missing == [] and unexpected == []
    assert isinstance(fresh.transformer_blocks[0].attn.to_q, LowRankLinear)
    assert fresh.transformer_blocks[0].attn.to_q.rank == 8
    layer = fresh.transformer_blocks[2].attn.to_k
    assert layer.qweight.dtype == torch.int8 and layer.wscale.dtype == torch.float32
    assert layer.keep_input is True
    assert fresh.transformer_blocks[0].attn.to_q.down.weight.dtype == torch.bfloat16
    assert fresh.proj.weight.dtype == torch.bfloat16
    for key, value in model.state_dict().items():
        got = fresh.state_dict()[key]
        if value.dtype in (torch.int8, torch.float32) and key.endswith(("qweight", "wscale")):
            assert torch.equal(got, value), key
        else:
            torch.testing.assert_close(got.float(), value.to(torch.bfloat16).float(), rtol=0, atol=0)


def test_sharded_partition_with_an_index(tmp_path):
    from hyperflow_h3_flash_amd.convert import load_partition, save_partition, shard_files

    model = filled_model(1)
    paths = save_partition(model, str(tmp_path), partition_config(), max_shard_bytes=8 << 10)
    assert len(paths) > 2 and (tmp_path / "diffusion_pytorch_model.safetensors.index.json").exists()
    assert shard_files(str(tmp_path)) == sorted(paths)
    fresh = Toy()
    load_partition(fresh, str(tmp_path))
    for key, value in model.state_dict().items():
        assert torch.equal(fresh.state_dict()[key], value), key
    # a shard the index lists is missing: refuse rather than load a partial model
    import os

    os.remove(paths[1])
    with pytest.raises(FileNotFoundError, match="missing"):
        load_partition(Toy(), str(tmp_path))


def test_partition_mismatches_are_reported(tmp_path):
    from hyperflow_h3_flash_amd.convert import load_partition, save_partition

    model = filled_model(2)
    save_partition(model, str(tmp_path), partition_config())
    # a model built without the quantization block has dense weights where the file has qweight/wscale
    with pytest.raises(RuntimeError, match="does not match"):
        load_partition(Toy(), str(tmp_path), prepare=False)
    missing, unexpected = load_partition(Toy(), str(tmp_path), prepare=False, strict=False)
    assert "transformer_blocks.2.attn.to_k.qweight" in unexpected
    assert "transformer_blocks.2.attn.to_k.weight" in missing
    bad = partition_config()
    bad["quantization"]["method"] = "fp8"
    save_partition(model, str(tmp_path / "bad"), bad)
    with pytest.raises(ValueError, match="unsupported quantization method"):
        load_partition(Toy(), str(tmp_path / "bad"))


def test_rank_padding_keeps_the_factors():
    """transformer.py:60-73 and 285-317: zero rows of down / columns of up; trimming restores the used rank."""
    from hyperflow_h3_flash_amd import LowRankLinear, set_lowrank_rank_multiple

    torch.manual_seed(0)
    model = nn.Module()
    model.a = LowRankLinear(64, 32, 8)
    model.b = LowRankLinear(64, 48, 16)
    model.b.down.weight.data[5:] = 0
    model.b.up.weight.data[:, 5:] = 0
    dense = {name: (m.up.weight @ m.down.weight).detach().clone() for name, m in (("a", model.a), ("b", model.b))}
    assert model.a.pad_rank(64) and not model.a.pad_rank(64)
    assert (model.a.rank, model.a.down.weight.shape, model.a.up.weight.shape) == (64, (64, 64), (32, 64))
    assert set_lowrank_rank_multiple(model, 8) == 2
    assert (model.a.rank, model.b.rank, model.b.down.out_features, model.b.up.in_features) == (8, 8, 8, 8)
    assert set_lowrank_rank_multiple(model, 8) == 0
    assert set_lowrank_rank_multiple(model, 0) == 1 and model.b.rank == 5
    for name, m in (("a", model.a), ("b", model.b)):
        torch.testing.assert_close(m.up.weight @ m.down.weight, dense[name], rtol=0, atol=0)


def test_fuse_qkv_checks_its_inputs():
    from hyperflow_h3_flash_amd import fuse_qkv

    a, b = Int8RotLinear(64, 32, 16), Int8RotLinear(64, 48, 16)
    fused = fuse_qkv(a, b)
    assert (fused.in_features, fused.out_features, fused.group) == (64, 80, 16)
    assert torch.equal(fused.qweight, torch.cat([a.qweight, b.qweight]))
    with pytest.raises(ValueError, match="in_features"):
        fuse_qkv(a, Int8RotLinear(128, 32, 16))
    with pytest.raises(ValueError, match="group"):
        fuse_qkv(a, Int8RotLinear(64, 32, 64))
    with pytest.raises(ValueError, match="rank"):
        fuse_qkv(a, Int8RotLinear(64, 32, 16, rank=8))
    with pytest.raises(ValueError):
        fuse_qkv()


class GELU(nn.Module):
    """Stand-in with the attributes of a feed-forward's tanh-GELU projection module: `proj`, then the activation."""

    def __init__(self, proj: nn.Module, approximate: str) -> None:
        super().__init__()
        self.proj, self.approximate = proj, approximate

    def forward(self, x):
        return nn.functional.gelu(self.proj(x), approximate=self.approximate)


def test_fuse_activations_folds_tanh_gelu_into_the_int8_projection():
    from hyperflow_h3_flash_amd.convert import fuse_activations

    up = Int8RotLinear(64, 128, group=16)
    ff = nn.Module()
    ff.net = nn.ModuleList([GELU(up, "tanh"), nn.Dropout(0.0), Int8RotLinear(128, 64, group=16)])
    ff.exact = GELU(Int8RotLinear(64, 128, group=16), "none")  # erf GELU: not the fused activation
    ff.dense = GELU(nn.Linear(64, 128), "tanh")  # not an INT8 projection
    names = fuse_activations(ff)
    assert names == ["net.0"]
    assert ff.net[0] is up and up.activation == "gelu_tanh"
    assert isinstance(ff.exact, GELU) and isinstance(ff.dense, GELU)
    assert ff.net[2].activation is None
    assert fuse_activations(ff) == []  # idempotent


class SwiGLU(nn.Module):
    """Stand-in with the attributes of a gated feed-forward's input module: `proj` (2F wide), then
    `hidden * silu(gate)` of its halves."""

    def __init__(self, proj: nn.Module) -> None:
        super().__init__()
        self.proj = proj

    def forward(self, x):
        hidden, gate = self.proj(x).chunk(2, dim=-1)
        return hidden * nn.functional.silu(gate)


def test_fuse_activations_folds_swiglu_into_the_int8_projection():
    from hyperflow_h3_flash_amd.convert import fuse_activations

    up = Int8RotLinear(64, 256, group=16)
    ff = nn.Module()
    ff.net = nn.ModuleList([SwiGLU(up), nn.Dropout(0.0), Int8RotLinear(128, 64, group=16)])
    ff.odd = SwiGLU(Int8RotLinear(64, 80, group=16))  # halves of 40: not a multiple of 16, stays unfused
    ff.dense = SwiGLU(nn.Linear(64, 256))  # not an INT8 projection
    names = fuse_activations(ff)
    assert names == ["net.0"]
    assert ff.net[0] is up and up.activation == "swiglu"
    assert isinstance(ff.odd, SwiGLU) and isinstance(ff.dense, SwiGLU)
    assert "activation=swiglu" in repr(up)
    assert fuse_activations(ff) == []


def test_gated_activation_needs_a_width_divisible_by_32():
    with pytest.raises(ValueError, match="32"):
        Int8RotLinear(64, 80, group=16, activation="swiglu")
    Int8RotLinear(64, 96, group=16, activation="swiglu_gate_first")
