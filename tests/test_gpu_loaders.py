"""Checkpoints loaded by the two readers, run on the HIP path against the oracle.

The partition format (config.json + safetensors shards, transformer.py:185-203) and the ComfyUI single-file layout
(integrations/ComfyUI-HyperFlow-Flash/safetensors_io.py:18-58, model_patch.py:27-32,60-63) are read on the CPU
by `convert.load_partition` and `comfy.load_comfy_checkpoint`; here the loaded layers run on the device and are
compared with the oracle evaluated on the tensors as the FILE holds them, so a mistake in the mapping (a swapped
gated half, a scale broadcast wrongly, a transposed factor) shows. Bars: INT8 layers bitwise the oracle's
`convrot_linear` (rank 0, no bias: the reference's own arithmetic); the gated projection's SwiGLU bitwise the
oracle's SwiGLU of ComfyUI's (gate, hidden) output order; low-rank layers within the fp32-sum bound of the oracle's
exactly rounded products at each of the two stages and bitwise the oracle's chain `up(down(x))` on >= 98 % of the
elements (the device sums in fp32).
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from golden_utils import within_fp32_sum_bound
from torch import nn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
G = 256
D, FFN, M = 512, 768, 96


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


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return bits_of(t.to(torch.bfloat16))


def check_lowrank(lib, layer, x_bits, down_bits, up_bits):
    """The loaded low-rank layer against the file's factors: its intermediate u (the same kernel call the forward
    makes) within the fp32-sum bound of the oracle's exactly rounded ``bf16(x @ down^T)``, its output within the
    fp32-sum bound of the oracle's ``bf16(u @ up^T)`` of that u, and >= 98 % of the outputs bitwise the oracle's
    chain on the file's tensors."""
    from hyperflow_h3_flash_amd.int8 import lowrank_down

    x = to_dev_bf16(x_bits)
    with torch.no_grad():
        y = layer(x)
        u = lowrank_down(x, layer.down.weight)
    torch.cuda.synchronize()
    u_bits = bits_of(u)
    f32 = lib.bf16_to_f32
    assert within_fp32_sum_bound(f32(u_bits), f32(lib.lowrank_down(x_bits, down_bits)), f32(x_bits), f32(down_bits))
    assert within_fp32_sum_bound(f32(bits_of(y)), f32(lib.lowrank_up(u_bits, up_bits)), f32(u_bits), f32(up_bits))
    chain = lib.lowrank_up(lib.lowrank_down(x_bits, down_bits), up_bits)
    assert (bits_of(y) == chain).mean() > 0.98


def run_int8(layer, x_bits):
    with torch.no_grad():
        y = layer(to_dev_bf16(x_bits))
    torch.cuda.synchronize()
    return bits_of(y)


# ---------------------------------------------------------------------------------------------- partition format


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
    def __init__(self):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([Block(D, FFN) for _ in range(2)])


PARTITION = {
    "lowrank_ranks": {"transformer_blocks.0.attn.to_q": 32, "transformer_blocks.1.ff.net.2": 64},
    "quantization": {"method": "int8_convrot", "group": G,
                     "linears": ["transformer_blocks.0.attn.to_k", "transformer_blocks.0.ff.net.0",
                                 "transformer_blocks.1.attn.to_out.0", "transformer_blocks.1.ff.net.0"]},
    "dropped_blocks": [],
}


def test_partition_round_trip_runs_the_oracles_layers(oracle_lib, tmp_path):
    from hyperflow_h3_flash_amd import Int8RotLinear, LowRankLinear
    from hyperflow_h3_flash_amd.convert import load_partition, load_quantized, prepare_model, save_partition

    torch.manual_seed(11)
    model = prepare_model(Toy(), PARTITION)
    for module in model.modules():
        if isinstance(module, Int8RotLinear):
            load_quantized(module, torch.randn(module.out_features, module.in_features) * 0.02)
        elif isinstance(module, LowRankLinear):
            with torch.no_grad():
                module.down.weight.copy_(torch.randn_like(module.down.weight) * 0.02)
                module.up.weight.copy_(torch.randn_like(module.up.weight) * 0.02)
    paths = save_partition(model, str(tmp_path), PARTITION, max_shard_bytes=256 << 10)
    assert len(paths) > 1  # sharded, with an index
    fresh = Toy().to(torch.bfloat16)
    missing, unexpected = load_partition(fresh, str(tmp_path))
    assert missing == [] and unexpected == []
    fresh = fresh.to(DEV)
    # the file's tensors, read back independently of the loader
    from safetensors.torch import load_file

    stored = {}
    for path in paths:
        stored.update(load_file(path))
    int8_names = PARTITION["quantization"]["linears"]
    for i, name in enumerate(int8_names):
        layer = fresh.get_submodule(name)
        assert isinstance(layer, Int8RotLinear) and layer.qweight.device.type == "cuda"
        x = oracle_lib.make_inputs(M, layer.in_features, 8, G, outlier_frac=0.01, outlier_scale=20.0,
                                   seed=100 + i)["x"]
        w = stored[f"{name}.qweight"].numpy()
        ws = stored[f"{name}.wscale"].numpy()
        assert w.dtype == np.int8 and ws.dtype == np.float32
        ref = oracle_lib.convrot_linear(x, w, ws, G)
        np.testing.assert_array_equal(run_int8(layer, x), ref["y"])
    for i, (name, rank) in enumerate(PARTITION["lowrank_ranks"].items()):
        layer = fresh.get_submodule(name)
        assert isinstance(layer, LowRankLinear) and layer.rank == rank
        x = oracle_lib.make_inputs(M, layer.down.weight.shape[1], 8, G, seed=200 + i)["x"]
        check_lowrank(oracle_lib, layer, x, bf16_bits(stored[f"{name}.down.weight"]),
                      bf16_bits(stored[f"{name}.up.weight"]))


# ------------------------------------------------------------------------------------------- ComfyUI layout


class GatedProj(nn.Module):
    def __init__(self, d, ffn):
        super().__init__()
        self.proj = nn.Linear(d, 2 * ffn, bias=False)


class ComfyBlock(nn.Module):
    def __init__(self, d, ffn):
        super().__init__()
        self.attn = Attn(d)
        self.ff = nn.Module()
        self.ff.net = nn.ModuleList([GatedProj(d, ffn), nn.Dropout(0.0), nn.Linear(ffn, d, bias=False)])


class ComfyToy(nn.Module):
    def __init__(self):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([ComfyBlock(D, FFN)])


def quant_tag():
    return torch.tensor(list(json.dumps({"format": "int8_tensorwise"}).encode()), dtype=torch.uint8)


def test_comfy_layout_runs_the_oracles_layers(oracle_lib, tmp_path):
    """A synthetic ComfyUI-layout file: q_proj INT8 with per-channel scales, out_proj INT8 with a one-element scale,
    the gated fc1 INT8 in ComfyUI's (gate, hidden) row order, k_proj and fc2 low-rank."""
    from safetensors.torch import save_file

    from hyperflow_h3_flash_amd import Int8RotLinear, LowRankLinear
    from hyperflow_h3_flash_amd.comfy import load_comfy_checkpoint

    gen = torch.Generator().manual_seed(5)
    t = {}

    def int8(prefix, n, k, scalar=False):
        t[f"{prefix}.weight"] = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=gen)
        t[f"{prefix}.weight_scale"] = (torch.tensor([4e-3]) if scalar else
                                       torch.rand(n, generator=gen) * 9e-3 + 1e-3)
        t[f"{prefix}.comfy_quant"] = quant_tag()

    def lowrank(prefix, n, k, r):
        t[f"{prefix}.down.weight"] = (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16)
        t[f"{prefix}.up.weight"] = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16)

    int8("blocks.0.attn.q_proj", D, D)
    int8("blocks.0.attn.out_proj", D, D, scalar=True)
    int8("blocks.0.mlp.fc1", 2 * FFN, D)
    lowrank("blocks.0.attn.k_proj", D, D, 32)
    lowrank("blocks.0.mlp.fc2", D, FFN, 64)
    path = tmp_path / "model.safetensors"
    save_file(t, str(path), metadata={"hyperflow": json.dumps({"format": 1, "convrot_group": G})})

    model = ComfyToy()
    done = load_comfy_checkpoint(model, str(path), group=G)
    assert len(done["int8"]) == 3 and len(done["lowrank"]) == 2
    model = model.to(DEV)
    blk = model.transformer_blocks[0]
    x = oracle_lib.make_inputs(M, D, 8, G, outlier_frac=0.01, outlier_scale=20.0, seed=31)["x"]

    # per-channel scales
    q = blk.attn.to_q
    assert isinstance(q, Int8RotLinear)
    ref = oracle_lib.convrot_linear(x, t["blocks.0.attn.q_proj.weight"].numpy(),
                                    t["blocks.0.attn.q_proj.weight_scale"].numpy(), G)
    np.testing.assert_array_equal(run_int8(q, x), ref["y"])
    # a one-element scale broadcast over the output channels
    ref = oracle_lib.convrot_linear(x, t["blocks.0.attn.out_proj.weight"].numpy(),
                                    np.full(D, 4e-3, dtype=np.float32), G)
    np.testing.assert_array_equal(run_int8(blk.attn.to_out[0], x), ref["y"])
    # the gated projection: ComfyUI's rows are (gate, hidden); the loaded module's output is (hidden, gate)
    proj = blk.ff.net[0].proj
    file_order = oracle_lib.convrot_linear(x, t["blocks.0.mlp.fc1.weight"].numpy(),
                                           t["blocks.0.mlp.fc1.weight_scale"].numpy(), G)["y"]
    got = run_int8(proj, x)
    np.testing.assert_array_equal(got[:, :FFN], file_order[:, FFN:])
    np.testing.assert_array_equal(got[:, FFN:], file_order[:, :FFN])
    proj.activation = "swiglu"
    np.testing.assert_array_equal(run_int8(proj, x), oracle_lib.swiglu(file_order, gate_first=True))
    # low-rank parts
    assert isinstance(blk.attn.to_k, LowRankLinear) and isinstance(blk.ff.net[2], LowRankLinear)
    blk.attn.to_k.to(torch.bfloat16)
    blk.ff.net[2].to(torch.bfloat16)
    check_lowrank(oracle_lib, blk.attn.to_k, x, bf16_bits(t["blocks.0.attn.k_proj.down.weight"]),
                  bf16_bits(t["blocks.0.attn.k_proj.up.weight"]))
    x2 = oracle_lib.make_inputs(M, FFN, 8, G, seed=32)["x"]
    check_lowrank(oracle_lib, blk.ff.net[2], x2, bf16_bits(t["blocks.0.mlp.fc2.down.weight"]),
                  bf16_bits(t["blocks.0.mlp.fc2.up.weight"]))
