"""Putting `Int8RotLinear` into a model: the config seam of the reference transformer and its checkpoint format.

* `replace_linear` — swap one bias-free ``nn.Linear`` for another module built from its shape
  (src/hyperflow_h3_flash/transformer.py:112-122), TypeError for anything else.
* `apply_quantization` — the ``config.json`` ``quantization`` block: ``{"method": "int8_convrot", "group": G,
  "linears": [dotted names]}`` (transformer.py:194-198), ValueError for another method, and ``keep_input`` on
  ``attn.to_q`` / ``attn.to_k`` so Q, K and V share one quantized input (transformer.py:199-203).
* `quantize_weight` — the checkpoint format ``qweight = round(W R / wscale)``, ``wscale = absmax_row(W R) / 127``,
  computed in float64 (tests/test_int8.py:31-36). An offline conversion step for bf16/fp32 weights, not part of the
  forward pass.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor, nn

from .int8 import Int8RotLinear, regular_hadamard

METHOD = "int8_convrot"


def replace_linear(model: nn.Module, name: str, make: type[nn.Module], *args: Any, **kwargs: Any) -> nn.Module:
    """Replace the bias-free ``nn.Linear`` at dotted path ``name`` by ``make(in_features, out_features, *args)``."""
    owner_name, _, attr = name.rpartition(".")
    owner = model.get_submodule(owner_name) if owner_name else model
    dense = owner[int(attr)] if isinstance(owner, nn.ModuleList) else getattr(owner, attr)
    if type(dense) is not nn.Linear or dense.bias is not None:
        raise TypeError(f"{name} is not a bias-free nn.Linear")
    replacement = make(dense.in_features, dense.out_features, *args, **kwargs)
    if isinstance(owner, nn.ModuleList):
        owner[int(attr)] = replacement
    else:
        setattr(owner, attr, replacement)
    return replacement


def apply_quantization(model: nn.Module, quantization: dict[str, Any] | None) -> list[str]:
    """Replace every linear the ``quantization`` block names by `Int8RotLinear`; returns the replaced names."""
    if not quantization:
        return []
    if quantization.get("method") != METHOD:
        raise ValueError(f"unsupported quantization method {quantization.get('method')!r}")
    group = int(quantization["group"])
    names = list(quantization["linears"])
    for name in names:
        replace_linear(model, name, Int8RotLinear, group)
    for module in model.modules():
        for attr in ("to_q", "to_k"):
            layer = getattr(module, attr, None)
            if isinstance(layer, Int8RotLinear):
                layer.keep_input = True
    return names


@torch.no_grad()
def quantize_weight(weight: Tensor, group: int) -> tuple[Tensor, Tensor]:
    """``(qweight int8 [N, K], wscale fp32 [N])`` for a dense weight [N, K], in float64 on the weight's device."""
    w = weight.detach().to(torch.float64)
    n, k = w.shape
    if k % group:
        raise ValueError(f"in_features {k} is not a multiple of the Hadamard group {group}")
    h = regular_hadamard(group).to(device=w.device, dtype=torch.float64)
    rotated = (w.reshape(n, k // group, group) @ h).reshape(n, k)
    wscale = rotated.abs().amax(1) / 127.0
    qweight = (rotated / wscale[:, None]).round().clamp(-127, 127).to(torch.int8)
    return qweight, wscale.float()


@torch.no_grad()
def load_quantized(layer: Int8RotLinear, weight: Tensor) -> Int8RotLinear:
    """Fill ``layer`` from a dense weight with `quantize_weight`."""
    qweight, wscale = quantize_weight(weight, layer.group)
    layer.qweight.copy_(qweight.to(layer.qweight.device))
    layer.wscale.copy_(wscale.to(layer.wscale.device))
    return layer


__all__ = ["METHOD", "apply_quantization", "load_quantized", "quantize_weight", "replace_linear"]
