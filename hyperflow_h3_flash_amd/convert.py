"""Putting `Int8RotLinear` into a model: the config seam of the reference transformer and its checkpoint format.

* `replace_linear` — swap one bias-free ``nn.Linear`` for another module built from its shape
  (src/hyperflow_h3_flash/transformer.py:112-122), TypeError for anything else.
* `apply_quantization` — the ``config.json`` ``quantization`` block: ``{"method": "int8_convrot", "group": G,
  "linears": [dotted names]}`` (transformer.py:194-198), ValueError for another method, and ``keep_input`` on
  ``attn.to_q`` / ``attn.to_k`` so Q, K and V share one quantized input (transformer.py:199-203).
* `fuse_activations` — fold a feed-forward's tanh-GELU or SwiGLU module into its `Int8RotLinear` projection's
  epilogue.
* `quantize_weight` — the checkpoint format ``qweight = round(W R / wscale)``, ``wscale = absmax_row(W R) / 127``,
  computed in float64 (tests/test_int8.py:31-36). An offline conversion step for bf16/fp32 weights, not part of the
  forward pass.
* `prepare_model` / `load_partition` / `save_partition` — a checkpoint partition such as ``fl2va_int8_convrot``: a
  folder with ``config.json`` (its ``lowrank_ranks`` and ``quantization`` blocks build the layers,
  transformer.py:185-203) and safetensors shards (an optional ``*.safetensors.index.json`` lists them). Tensors are
  read with the safetensors loader, which executes nothing from the file. ``qweight`` stays int8 and ``wscale``
  stays fp32 whatever the model's dtype, as the reference's ``_keep_in_fp32_modules`` keeps them
  (transformer.py:129-133, tests/test_transformer.py:164-175); other floating tensors take the model's dtype.
"""

from __future__ import annotations

import json
import os
from typing import Any

import torch
from torch import Tensor, nn

from .int8 import Int8RotLinear, regular_hadamard
from .lowrank import LowRankLinear

METHOD = "int8_convrot"


def replace_linear(model: nn.Module, name: str, make: type[nn.Module], *args: Any, **kwargs: Any) -> nn.Module:
    """Replace the bias-free ``nn.Linear`` at dotted path ``name`` by ``make(in_features, out_features, *args)``."""
    owner_name, _, attr = name.rpartition(".")
    owner = model.get_submodule(owner_name) if owner_name else model
    dense = owner[int(attr)] if isinstance(owner, nn.ModuleList) else getattr(owner, attr)
    if type(dense) is not nn.Linear or dense.bias is not None:
        raise TypeError(f"{name} is not a bias-free nn.Linear")
    replacement = make(dense.in_features, dense.out_features, *args, **kwargs).to(dense.weight.device)
    if isinstance(replacement, LowRankLinear):
        replacement.to(dense.weight.dtype)  # the factors take the model's dtype; INT8 storage dtypes are fixed
    if isinstance(owner, nn.ModuleList):
        owner[int(attr)] = replacement
    else:
        setattr(owner, attr, replacement)
    return replacement


def fuse_activations(model: nn.Module) -> list[str]:
    """Fold every feed-forward activation module whose projection is an `Int8RotLinear` into that linear's GEMM
    epilogue (the feed-forward's first ``net`` entry, transformer.py:75-99), replacing the module by its ``proj``:

    * a ``GELU`` module with ``approximate == "tanh"`` (forward ``gelu(proj(x))``) -> ``activation="gelu_tanh"``;
    * a ``SwiGLU`` module (forward ``h, g = proj(x).chunk(2, -1); h * silu(g)``, the model's gated feed-forward)
      -> ``activation="swiglu"``, when its projection's width is a multiple of 32.

    Returns the replaced modules' names."""
    found = []
    for name, module in model.named_modules():
        proj = getattr(module, "proj", None)
        if not isinstance(proj, Int8RotLinear) or proj.activation is not None:
            continue
        kind = type(module).__name__
        if kind == "GELU" and getattr(module, "approximate", None) == "tanh":
            found.append((name, "gelu_tanh"))
        elif kind == "SwiGLU" and proj.out_features % 32 == 0:
            found.append((name, "swiglu"))
    for name, activation in found:
        owner_name, _, attr = name.rpartition(".")
        owner = model.get_submodule(owner_name) if owner_name else model
        act = owner[int(attr)] if isinstance(owner, nn.ModuleList) else getattr(owner, attr)
        act.proj.activation = activation
        if isinstance(owner, nn.ModuleList):
            owner[int(attr)] = act.proj
        else:
            setattr(owner, attr, act.proj)
    return [name for name, _ in found]


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


CONFIG_NAME = "config.json"
#: Leaves stored in their own dtype whatever the model's (int8 codes, fp32 per-channel scales).
STORAGE_DTYPE_LEAVES = ("qweight", "wscale")


def read_config(folder: str) -> dict[str, Any]:
    with open(os.path.join(folder, CONFIG_NAME)) as f:
        return json.load(f)


def prepare_model(model: nn.Module, config: dict[str, Any]) -> nn.Module:
    """Build the compressed layers a partition's ``config.json`` names: `LowRankLinear` for every entry of
    ``lowrank_ranks`` and `Int8RotLinear` for the ``quantization`` block (transformer.py:185-203)."""
    for name, rank in (config.get("lowrank_ranks") or {}).items():
        replace_linear(model, name, LowRankLinear, int(rank))
    apply_quantization(model, config.get("quantization"))
    return model


def shard_files(folder: str) -> list[str]:
    """The partition's safetensors shards: those its index lists (all must exist), else every ``*.safetensors``."""
    indexes = sorted(f for f in os.listdir(folder) if f.endswith(".safetensors.index.json"))
    if indexes:
        files: list[str] = []
        for index in indexes:
            with open(os.path.join(folder, index)) as f:
                files += sorted(set(json.load(f)["weight_map"].values()))
        missing = [f for f in files if not os.path.isfile(os.path.join(folder, f))]
        if missing:
            raise FileNotFoundError(f"{folder}: shards listed in the index are missing: {missing}")
        return [os.path.join(folder, f) for f in files]
    files = sorted(f for f in os.listdir(folder) if f.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"{folder}: no safetensors shards")
    return [os.path.join(folder, f) for f in files]


@torch.no_grad()
def load_partition(model: nn.Module, folder: str, *, prepare: bool = True, strict: bool = True,
                   dtype: torch.dtype | None = None) -> tuple[list[str], list[str]]:
    """Load a checkpoint partition into ``model`` (built by `prepare_model` from its ``config.json`` first unless
    ``prepare=False``). Returns ``(missing, unexpected)`` keys; with ``strict`` either being non-empty raises.

    Every tensor lands on the device of the parameter or buffer it replaces. ``qweight`` and ``wscale`` keep their
    storage dtypes; other floating tensors are cast to ``dtype`` (default: the replaced tensor's dtype)."""
    from safetensors.torch import load_file

    if prepare:
        prepare_model(model, read_config(folder))
    targets = dict(model.named_parameters())
    targets.update(dict(model.named_buffers()))
    seen: set[str] = set()
    unexpected: list[str] = []
    for path in shard_files(folder):
        for key, tensor in load_file(path, device="cpu").items():
            if key not in targets:
                unexpected.append(key)
                continue
            current = targets[key]
            if tuple(current.shape) != tuple(tensor.shape):
                raise ValueError(f"{key}: checkpoint shape {tuple(tensor.shape)} != model {tuple(current.shape)}")
            leaf = key.rpartition(".")[2]
            if leaf in STORAGE_DTYPE_LEAVES or not tensor.is_floating_point():
                target_dtype = tensor.dtype
            else:
                target_dtype = dtype or current.dtype
            value = tensor.to(device=current.device, dtype=target_dtype)
            owner_name, _, attr = key.rpartition(".")
            owner = model.get_submodule(owner_name) if owner_name else model
            if attr in owner._parameters:
                owner._parameters[attr] = nn.Parameter(value, requires_grad=current.requires_grad)
            else:
                owner._buffers[attr] = value
            seen.add(key)
    missing = sorted(set(targets) - seen)
    if strict and (missing or unexpected):
        raise RuntimeError(f"checkpoint does not match the model: missing {missing}, unexpected {unexpected}")
    return missing, unexpected


def save_partition(model: nn.Module, folder: str, config: dict[str, Any], *, max_shard_bytes: int = 5 << 30) -> list[str]:
    """Write ``config.json`` and the model's state dict as safetensors shards (with an index when there is more than
    one); returns the shard paths."""
    from safetensors.torch import save_file

    os.makedirs(folder, exist_ok=True)
    with open(os.path.join(folder, CONFIG_NAME), "w") as f:
        json.dump(config, f, indent=2, sort_keys=True)
    shards: list[dict[str, Tensor]] = [{}]
    size = 0
    for key, tensor in model.state_dict().items():
        nbytes = tensor.numel() * tensor.element_size()
        if shards[-1] and size + nbytes > max_shard_bytes:
            shards.append({})
            size = 0
        shards[-1][key] = tensor.detach().to("cpu").contiguous()
        size += nbytes
    names = (["diffusion_pytorch_model.safetensors"] if len(shards) == 1 else
             [f"diffusion_pytorch_model-{i + 1:05d}-of-{len(shards):05d}.safetensors" for i in range(len(shards))])
    for name, shard in zip(names, shards):
        save_file(shard, os.path.join(folder, name))
    if len(shards) > 1:
        weight_map = {key: name for name, shard in zip(names, shards) for key in shard}
        with open(os.path.join(folder, "diffusion_pytorch_model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": weight_map}, f, indent=2, sort_keys=True)
    return [os.path.join(folder, n) for n in names]


__all__ = ["CONFIG_NAME", "METHOD", "apply_quantization", "fuse_activations", "load_partition", "load_quantized",
           "prepare_model", "quantize_weight", "read_config", "replace_linear", "save_partition", "shard_files"]
