"""The ComfyUI-layout HyperFlow checkpoint reader (integrations/ComfyUI-HyperFlow-Flash/safetensors_io.py:18-58,
model_patch.py:27-32) on synthetic files: the metadata check, the key map onto the reference model's names, the
gate/hidden half order of the gated projection, and the comfy_quant check. CPU only."""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file
from torch import nn

from hyperflow_h3_flash_amd import Int8RotLinear, LowRankLinear
from hyperflow_h3_flash_amd.comfy import check_metadata, decode_comfy_quant, load_comfy_checkpoint


class GatedProj(nn.Module):
    def __init__(self, d, ffn):
        super().__init__()
        self.proj = nn.Linear(d, 2 * ffn, bias=False)


class Block(nn.Module):
    def __init__(self, d, ffn):
        super().__init__()
        self.attn = nn.Module()
        for name in ("to_q", "to_k", "to_v"):
            setattr(self.attn, name, nn.Linear(d, d, bias=False))
        self.attn.to_out = nn.ModuleList([nn.Linear(d, d, bias=False), nn.Dropout(0.0)])
        self.ff = nn.Module()
        self.ff.net = nn.ModuleList([GatedProj(d, ffn), nn.Dropout(0.0), nn.Linear(ffn, d, bias=False)])


class Toy(nn.Module):
    def __init__(self, d=64, ffn=96, blocks=2):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([Block(d, ffn) for _ in range(blocks)])


def quant_tag(fmt="int8_tensorwise"):
    return torch.tensor(list(json.dumps({"format": fmt}).encode()), dtype=torch.uint8)


def int8_part(gen, n, k):
    return {"weight": torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=gen),
            "weight_scale": torch.rand(n, generator=gen) * 9e-3 + 1e-3, "comfy_quant": quant_tag()}


def write(path, tensors, metadata):
    save_file(tensors, str(path), metadata=metadata)


def comfy_file(tmp_path, fmt=1, scalar_scale=False, tag="int8_tensorwise", group=None):
    gen = torch.Generator().manual_seed(7)
    d, ffn = 64, 96
    t = {}
    for leaf, v in int8_part(gen, d, d).items():
        t[f"blocks.0.attn.q_proj.{leaf}"] = v
    t["blocks.0.attn.k_proj.down.weight"] = (torch.randn(8, d, generator=gen) * 0.02).to(torch.bfloat16)
    t["blocks.0.attn.k_proj.up.weight"] = (torch.randn(d, 8, generator=gen) * 0.02).to(torch.bfloat16)
    for leaf, v in int8_part(gen, 2 * ffn, d).items():
        t[f"blocks.1.mlp.fc1.{leaf}"] = v
    out = int8_part(gen, d, d)
    if scalar_scale:
        out["weight_scale"] = torch.tensor([3e-3])
    out["comfy_quant"] = quant_tag(tag)
    for leaf, v in out.items():
        t[f"blocks.1.attn.out_proj.{leaf}"] = v
    t["blocks.1.mlp.fc2.down.weight"] = (torch.randn(16, ffn, generator=gen) * 0.02).to(torch.bfloat16)
    t["blocks.1.mlp.fc2.up.weight"] = (torch.randn(d, 16, generator=gen) * 0.02).to(torch.bfloat16)
    t["final_norm.weight"] = torch.ones(d)
    path = tmp_path / "model.safetensors"
    meta = {"format": fmt} if group is None else {"format": fmt, "convrot_group": group}
    write(path, t, {"hyperflow": json.dumps(meta)})
    return path, t


def test_metadata_check(tmp_path):
    path, _ = comfy_file(tmp_path)
    assert check_metadata(str(path))["format"] == 1
    plain = tmp_path / "plain.safetensors"
    write(plain, {"w": torch.zeros(2)}, {})
    with pytest.raises(RuntimeError, match="no 'hyperflow' entry"):
        check_metadata(str(plain))
    future = tmp_path / "future.safetensors"
    write(future, {"w": torch.zeros(2)}, {"hyperflow": json.dumps({"format": 2})})
    with pytest.raises(RuntimeError, match="format 2"):
        check_metadata(str(future))


def test_block_linears_land_on_the_reference_names(tmp_path):
    path, t = comfy_file(tmp_path)
    model = Toy()
    done = load_comfy_checkpoint(model, str(path), group=16, rotated=True)
    b0, b1 = model.transformer_blocks
    assert sorted(done["int8"]) == ["transformer_blocks.0.attn.to_q", "transformer_blocks.1.attn.to_out.0",
                                    "transformer_blocks.1.ff.net.0.proj"]
    assert sorted(done["lowrank"]) == ["transformer_blocks.0.attn.to_k", "transformer_blocks.1.ff.net.2"]
    assert done["skipped"] == ["final_norm.weight"]
    assert isinstance(b0.attn.to_q, Int8RotLinear) and isinstance(b0.attn.to_k, LowRankLinear)
    assert isinstance(b0.attn.to_v, nn.Linear) and not isinstance(b0.attn.to_v, (Int8RotLinear, LowRankLinear))
    assert torch.equal(b0.attn.to_q.qweight, t["blocks.0.attn.q_proj.weight"])
    assert torch.equal(b0.attn.to_q.wscale, t["blocks.0.attn.q_proj.weight_scale"])
    assert b0.attn.to_q.comfy_quant == {"format": "int8_tensorwise"}
    assert torch.equal(b0.attn.to_k.down.weight, t["blocks.0.attn.k_proj.down.weight"].float())
    assert torch.equal(b1.ff.net[2].up.weight, t["blocks.1.mlp.fc2.up.weight"].float())


def test_gated_projection_halves_follow_the_reference_order(tmp_path):
    """ComfyUI's fc1 output is (gate, hidden); the loaded ff.net.0.proj is (hidden, gate), so SwiGLU on it equals
    ComfyUI's silu(gate) * hidden of the file's own row order."""
    path, t = comfy_file(tmp_path)
    model = Toy()
    load_comfy_checkpoint(model, str(path), group=16, rotated=True)
    proj = model.transformer_blocks[1].ff.net[0].proj
    comfy = Int8RotLinear(64, 192, 16, activation="swiglu_gate_first")
    comfy.qweight.copy_(t["blocks.1.mlp.fc1.weight"])
    comfy.wscale.copy_(t["blocks.1.mlp.fc1.weight_scale"])
    x = torch.randn(5, 64).to(torch.bfloat16)
    proj.activation = "swiglu"
    assert torch.equal(proj(x), comfy(x))
    proj.activation = None
    comfy.activation = None
    gate_c, hidden_c = comfy(x).chunk(2, dim=-1)
    hidden, gate = proj(x).chunk(2, dim=-1)
    assert torch.equal(hidden, hidden_c) and torch.equal(gate, gate_c)


def test_scalar_scale_is_broadcast_and_format_tag_checked(tmp_path):
    path, _ = comfy_file(tmp_path, scalar_scale=True)
    model = Toy()
    load_comfy_checkpoint(model, str(path), group=16, rotated=True)
    ws = model.transformer_blocks[1].attn.to_out[0].wscale
    assert ws.shape == (64,) and torch.all(ws == torch.tensor(3e-3, dtype=torch.float32))
    other = tmp_path / "other"
    other.mkdir()
    path2, _ = comfy_file(other, tag="fp8_tensorwise")
    with pytest.raises(ValueError, match="int8_tensorwise"):
        load_comfy_checkpoint(Toy(), str(path2), group=16, rotated=True)
    assert decode_comfy_quant(quant_tag()) == {"format": "int8_tensorwise"}


def test_int8_parts_need_a_stated_rotation_basis(tmp_path):
    """Int8RotLinear rotates its input, so INT8 weights load only when the file's metadata names their Hadamard group
    or the caller vouches for it; low-rank parts alone load either way."""
    path, t = comfy_file(tmp_path)
    with pytest.raises(ValueError, match="rotated=True"):
        load_comfy_checkpoint(Toy(), str(path), group=16)
    named = tmp_path / "named"
    named.mkdir()
    path2, _ = comfy_file(named, group=16)
    model = Toy()
    done = load_comfy_checkpoint(model, str(path2), group=16)
    assert len(done["int8"]) == 3
    assert torch.equal(model.transformer_blocks[0].attn.to_q.qweight, t["blocks.0.attn.q_proj.weight"])
    with pytest.raises(ValueError, match="group 16, loader asked for 64"):
        load_comfy_checkpoint(Toy(), str(path2), group=64)
