"""The low-rank linear of the reference transformer on the gfx950 kernels, and the fused Q/K/V projection.

* `LowRankLinear` — ``y = up(down(x))``, the factorized replacement of a bias-free ``nn.Linear``
  (src/hyperflow_h3_flash/transformer.py:48-72): the same constructor, ``down.weight`` [rank, in] and
  ``up.weight`` [out, rank] parameters and ``pad_rank``. For bf16 device inputs both products run on the HIP
  kernels (``hf_lowrank_down``, then ``hf_lowrank_up``) with the reference's bf16 intermediate:
  ``bf16(bf16(x @ down^T) @ up^T)``, each sum in fp32 and rounded once.
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


def _round_up(value: int, multiple: int) -> int:
    return value if multiple <= 0 else (value + multiple - 1) // multiple * multiple


def _resize_rank(layer: "LowRankLinear", rank: int) -> None:
    """Give ``layer`` exactly ``rank`` ranks: drop trailing rows of ``down`` / columns of ``up``, or append zero ones.
    Zero ranks contribute exact zeros to ``up @ down``, so the layer's function is unchanged whenever only zero
    ranks are dropped."""
    grow = rank - layer.rank
    down, up = layer.down.weight.detach(), layer.up.weight.detach()
    if grow >= 0:
        down = torch.nn.functional.pad(down, (0, 0, 0, grow))
        up = torch.nn.functional.pad(up, (0, grow))
    else:
        down, up = down[:rank], up[:, :rank]
    layer.down.weight = nn.Parameter(down.contiguous(), requires_grad=False)
    layer.up.weight = nn.Parameter(up.contiguous(), requires_grad=False)
    layer.rank = layer.down.out_features = layer.up.in_features = rank


class LowRankLinear(nn.Module):
    """A bias-free linear stored as two factors, ``y = up(down(x))`` with ``down.weight`` [rank, in] and
    ``up.weight`` [out, rank] (the reference's module, transformer.py:48-72).

    bf16 inputs on a ROCm device run the two HIP products (``hf_lowrank_down``, ``hf_lowrank_up``): each sum in fp32,
    rounded once to bf16 like the bf16 ``nn.Linear``s they replace. Every other case (host tensors, or a float32 /
    float64 module) is the reference's own ``up(down(x))`` in the input's dtype."""

    def __init__(self, in_features: int, out_features: int, rank: int) -> None:
        super().__init__()
        self.in_features, self.out_features, self.rank = in_features, out_features, rank
        self.down = nn.Linear(in_features, rank, bias=False)
        self.up = nn.Linear(rank, out_features, bias=False)

    def _on_kernels(self, x: Tensor) -> bool:
        return (x.is_cuda and x.dtype == torch.bfloat16 and self.down.weight.dtype == torch.bfloat16
                and self.up.weight.dtype == torch.bfloat16 and self.in_features % 16 == 0)

    def forward(self, x: Tensor) -> Tensor:
        if not self._on_kernels(x):
            return self.up(self.down(x))
        kernels = _kernels()
        if kernels is None:
            raise RuntimeError(
                f"LowRankLinear on {x.device} needs the gfx950 HIP library; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`"
            )
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).contiguous()
        u = kernels.lowrank_down(x2, self.down.weight)
        y = kernels.lowrank_up(u, self.up.weight)
        return y.reshape(*shape[:-1], self.out_features)

    @torch.no_grad()
    def pad_rank(self, multiple: int = RANK_MULTIPLE) -> bool:
        """Append zero ranks up to the next multiple of ``multiple`` (transformer.py:60-73); the product is
        unchanged. True when ranks were added."""
        target = _round_up(self.rank, multiple)
        if target == self.rank:
            return False
        _resize_rank(self, target)
        return True


def _used_rank(layer: LowRankLinear) -> int:
    """One past the last rank whose ``down`` row or ``up`` column holds a nonzero (at least 1): the rank before any
    zero padding (transformer.py:285-289)."""
    live = layer.down.weight.detach().ne(0).any(dim=1) | layer.up.weight.detach().ne(0).any(dim=0)
    ranks = torch.arange(1, live.numel() + 1, device=live.device)[live]
    return int(ranks.max()) if ranks.numel() else 1


@torch.no_grad()
def set_lowrank_rank_multiple(model: nn.Module, multiple: int) -> int:
    """Re-pad every `LowRankLinear` in ``model`` from its used rank up to a multiple of ``multiple`` (0 or less:
    the used rank itself), trimming or appending zero ranks; returns how many layers changed (transformer.py:292-317).

    The function computed is the same for every multiple. The kernels read the rank in chunks of 8, so multiples of 8
    need no padding per call."""
    layers = [m for m in model.modules() if isinstance(m, LowRankLinear)]
    resized = 0
    for layer in layers:
        target = _round_up(_used_rank(layer), multiple)
        if target != layer.rank:
            _resize_rank(layer, target)
            resized += 1
    return resized


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
