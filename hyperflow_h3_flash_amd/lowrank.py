"""The low-rank linear of the reference transformer on the gfx950 kernels, and the fused Q/K/V projection.

* `LowRankLinear` — ``y = up(down(x))``, the factorized replacement of a bias-free ``nn.Linear``
  (src/hyperflow_h3_flash/transformer.py:48-72): the same constructor, ``down.weight`` [rank, in] and
  ``up.weight`` [out, rank] parameters and ``pad_rank``. Both products run on the HIP kernels (``hf_lowrank_down``,
  then ``hf_lowrank_up``) with the reference's bf16 intermediate: ``bf16(bf16(x @ down^T) @ up^T)``, each sum in
  fp32 and rounded once.
* `set_lowrank_rank_multiple` — re-pad every low-rank linear of a model (transformer.py:285-317).
* `fuse_qkv` — one `Int8RotLinear` whose rows are the concatenated q, k and v weights. Q, K and V of a block read
  the same input (transformer.py:199-203), so one rotate + quantize and one GEMM produce exactly the three
  projections' outputs side by side: each output column depends only on its own weight row and scale.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from .int8 import Int8RotLinear, _kernels

#: Ranks are padded to multiples of this at load (transformer.py:45-46).
RANK_MULTIPLE = 64


class LowRankLinear(nn.Module):
    """``y = up(down(x))``, the factorized replacement of a bias-free `nn.Linear` (transformer.py:48-72)."""

    def __init__(self, in_features: int, out_features: int, rank: int) -> None:
        super().__init__()
        self.in_features, self.out_features, self.rank = in_features, out_features, rank
        self.down = nn.Linear(in_features, rank, bias=False)
        self.up = nn.Linear(rank, out_features, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).to(torch.bfloat16).contiguous()
        if not x2.is_cuda:
            raise RuntimeError(
                f"LowRankLinear runs on the gfx950 HIP kernels; move the module and its input to a ROCm device "
                f"(input is on {x2.device})"
            )
        kernels = _kernels()
        u = kernels.lowrank_down(x2, self.down.weight.to(torch.bfloat16))
        y = kernels.lowrank_up(u, self.up.weight.to(torch.bfloat16))
        return y.reshape(*shape[:-1], self.out_features).to(x.dtype)

    @torch.no_grad()
    def pad_rank(self, multiple: int = RANK_MULTIPLE) -> bool:
        """Zero-pad the rank up to a multiple of ``multiple``: the new rows of ``down`` and columns of ``up`` are
        zero, so ``up @ down`` is unchanged. Returns whether the rank changed (transformer.py:60-73)."""
        rank = -(-self.rank // multiple) * multiple
        if rank == self.rank:
            return False
        extra = rank - self.rank
        down, up = self.down.weight, self.up.weight
        self.down.weight = nn.Parameter(torch.cat([down, down.new_zeros(extra, down.shape[1])]), requires_grad=False)
        self.up.weight = nn.Parameter(torch.cat([up, up.new_zeros(up.shape[0], extra)], dim=1), requires_grad=False)
        self.down.out_features = self.up.in_features = self.rank = rank
        return True


def _used_rank(layer: LowRankLinear) -> int:
    """The rank without its zero padding (trailing zero rows of ``down`` and columns of ``up``)."""
    used = (layer.down.weight.detach().abs().amax(1) != 0) | (layer.up.weight.detach().abs().amax(0) != 0)
    nonzero = used.nonzero()
    return int(nonzero[-1]) + 1 if len(nonzero) else 1


@torch.no_grad()
def set_lowrank_rank_multiple(model: nn.Module, multiple: int) -> int:
    """Re-pad every `LowRankLinear` to a rank multiple of ``multiple`` (0: no padding); returns how many changed.

    Zero rows and columns add exact zeros, so every multiple computes the same function (transformer.py:292-317).
    The kernels read the rank in chunks of 8, so a multiple of 8 (or any multiple of it) avoids padding per call.
    """
    changed = 0
    for layer in model.modules():
        if not isinstance(layer, LowRankLinear):
            continue
        rank = _used_rank(layer)
        target = -(-rank // multiple) * multiple if multiple > 0 else rank
        if target == layer.rank:
            continue
        down, up = layer.down.weight.detach(), layer.up.weight.detach()
        if target < layer.rank:
            down, up = down[:target], up[:, :target]
        else:
            down = torch.cat([down, down.new_zeros(target - layer.rank, down.shape[1])])
            up = torch.cat([up, up.new_zeros(up.shape[0], target - layer.rank)], dim=1)
        layer.down.weight = nn.Parameter(down.contiguous(), requires_grad=False)
        layer.up.weight = nn.Parameter(up.contiguous(), requires_grad=False)
        layer.rank = layer.down.out_features = layer.up.in_features = target
        changed += 1
    return changed


@torch.no_grad()
def fuse_qkv(*layers: Int8RotLinear) -> Int8RotLinear:
    """One `Int8RotLinear` computing ``torch.cat([layer(x) for layer in layers], -1)`` bit for bit.

    The layers must read the same input width and share the Hadamard group; low-rank branches and biases are
    concatenated along the output too (the low-rank ranks must match, since they share the input projection)."""
    if not layers:
        raise ValueError("fuse_qkv needs at least one layer")
    first = layers[0]
    k, group, rank = first.in_features, first.group, first.rank
    for layer in layers:
        if layer.in_features != k or layer.group != group:
            raise ValueError("fused layers must share in_features and the Hadamard group")
        if layer.rank != rank or (layer.bias is None) != (first.bias is None):
            raise ValueError("fused layers must share the low-rank rank and the presence of a bias")
        if rank and not torch.equal(layer.down.weight, first.down.weight):
            raise ValueError("fused low-rank branches must share down.weight")
    n = sum(layer.out_features for layer in layers)
    fused = Int8RotLinear(k, n, group, rank=rank, bias=first.bias is not None).to(first.qweight.device)
    fused.qweight.copy_(torch.cat([layer.qweight for layer in layers]))
    fused.wscale.copy_(torch.cat([layer.wscale for layer in layers]))
    if rank:
        fused.down.weight.copy_(first.down.weight)
        fused.up.weight.copy_(torch.cat([layer.up.weight for layer in layers]))
    if first.bias is not None:
        fused.bias.copy_(torch.cat([layer.bias for layer in layers]))
    return fused


__all__ = ["RANK_MULTIPLE", "LowRankLinear", "fuse_qkv", "set_lowrank_rank_multiple"]
