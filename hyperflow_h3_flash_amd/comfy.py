"""Reading HyperFlow's ComfyUI-layout INT8 checkpoints into the drop-in modules.

The reference ships a second INT8 release for ComfyUI (integrations/ComfyUI-HyperFlow-Flash): one safetensors file
whose ``__metadata__`` carries a ``hyperflow`` JSON entry with the layout version in ``format`` (files without it
are not HyperFlow checkpoints; versions above 1 are newer than this reader, safetensors_io.py:18-58), and whose
block linears are named in ComfyUI's packed-DiT vocabulary (model_patch.py:27-32):

    blocks.<i>.<attn.q_proj | attn.k_proj | attn.v_proj | attn.out_proj | mlp.fc1 | mlp.fc2>.<leaf>

with leaves ``weight`` / ``weight_scale`` / ``comfy_quant`` for a dense (INT8 ``int8_tensorwise``) linear and
``down.weight`` / ``up.weight`` for a factorized (low-rank) one. This module maps them onto the reference model's
own names (``transformer_blocks.<i>.attn.to_q`` ... ``ff.net.2``):

* the INT8 ``weight`` (int8 [N, K]) becomes ``qweight`` and ``weight_scale`` becomes ``wscale`` (fp32 [N]; a
  one-element scale is broadcast over the N channels); ``comfy_quant`` (a uint8 tensor holding JSON) is decoded,
  must name the ``int8_tensorwise`` format, and is kept on the module as ``comfy_quant``;
* ``mlp.fc1`` is the gated up-projection, whose output ComfyUI splits as ``gate, hidden = fc1(x).chunk(2, -1)``
  (model_patch.py FactorizedMLP), while the reference model's ``ff.net.0.proj`` splits ``hidden, gate``: the two
  row halves (and their scales, or the rows of ``up``) are swapped so the module computes the reference's layout.

Not fixed by the reference tree (it lives in ComfyUI and comfy-kitchen, absent here): what ``int8_tensorwise``'s
scale multiplies and whether the released INT8 weights carry the block-Hadamard rotation of the convrot format. The
reader moves the tensors as they are into ``Int8RotLinear`` (which rotates its input with the module's ``group``)
only when the file's metadata names that group (``convrot_group``) or the caller vouches for the basis
(``rotated=True``); a checkpoint whose weights were not quantized in the rotated basis needs its own conversion.
"""

from __future__ import annotations

import json
import re
from collections import defaultdict
from typing import Any

import torch
from torch import Tensor, nn

from .convert import replace_linear
from .int8 import Int8RotLinear
from .lowrank import LowRankLinear

METADATA_KEY = "hyperflow"
SUPPORTED_FORMAT = 1
INT8_FORMAT = "int8_tensorwise"

#: ComfyUI block-linear tensor names (model_patch.py:27-32).
PART = re.compile(
    r"^blocks\.(\d+)\.(attn\.[qkv]_proj|attn\.out_proj|mlp\.fc[12])\."
    r"(down\.weight|up\.weight|weight|weight_scale|comfy_quant)$"
)

#: ComfyUI module name -> the reference model's module name inside ``transformer_blocks.<i>``.
MODULE_NAMES = {
    "attn.q_proj": "attn.to_q",
    "attn.k_proj": "attn.to_k",
    "attn.v_proj": "attn.to_v",
    "attn.out_proj": "attn.to_out.0",
    "mlp.fc1": "ff.net.0.proj",
    "mlp.fc2": "ff.net.2",
}


def hyperflow_metadata(path: str) -> dict[str, Any] | None:
    """The decoded ``hyperflow`` metadata of a safetensors file, or None when the file has none."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        metadata = f.metadata() or {}
    if METADATA_KEY not in metadata:
        return None
    return json.loads(metadata[METADATA_KEY])


def check_metadata(path: str) -> dict[str, Any]:
    """The file's ``hyperflow`` metadata; RuntimeError when it is missing or its ``format`` is newer than 1."""
    info = hyperflow_metadata(path)
    if info is None:
        raise RuntimeError(f"cannot read {path}: its safetensors header has no {METADATA_KEY!r} entry, so it is not "
                           "a HyperFlow INT8 file")
    version = int(info.get("format", 0))
    if version > SUPPORTED_FORMAT:
        raise RuntimeError(f"cannot read {path}: written in format {version}, and formats above {SUPPORTED_FORMAT} "
                           "are unknown to this loader")
    return info


def decode_comfy_quant(tensor: Tensor) -> dict[str, Any]:
    """The JSON dictionary a ``comfy_quant`` uint8 tensor holds."""
    raw = bytes(tensor.detach().to("cpu", torch.uint8).flatten().tolist())
    value = json.loads(raw.decode("utf-8"))
    if not isinstance(value, dict):
        raise ValueError(f"comfy_quant holds {type(value).__name__}, not a JSON object")
    return value


def group_parts(tensors: dict[str, Tensor]) -> tuple[dict[tuple[int, str], dict[str, Tensor]], list[str]]:
    """Block-linear tensors by (block, ComfyUI module), and the names that are not block linears."""
    parts: dict[tuple[int, str], dict[str, Tensor]] = defaultdict(dict)
    others = []
    for name, tensor in tensors.items():
        match = PART.match(name)
        if match is None:
            others.append(name)
        else:
            parts[int(match.group(1)), match.group(2)][match.group(3)] = tensor
    return dict(parts), others


def _swap_halves(t: Tensor) -> Tensor:
    half = t.shape[0] // 2
    if t.shape[0] != 2 * half:
        raise ValueError(f"a gated projection needs an even number of rows, got {t.shape[0]}")
    return torch.cat([t[half:], t[:half]])


def _module(model: nn.Module, name: str) -> nn.Module:
    owner_name, _, attr = name.rpartition(".")
    owner = model.get_submodule(owner_name) if owner_name else model
    return owner[int(attr)] if isinstance(owner, nn.ModuleList) else getattr(owner, attr)


#: Key of the ``hyperflow`` metadata entry that names the Hadamard group the INT8 weights were quantized in.
GROUP_KEY = "convrot_group"


@torch.no_grad()
def load_comfy_checkpoint(model: nn.Module, path: str, group: int, *, prefix: str = "transformer_blocks",
                          rotated: bool = False) -> dict[str, list[str]]:
    """Load the block linears of a ComfyUI-layout HyperFlow file into ``model`` (reference module names).

    Dense ``nn.Linear`` targets are replaced by `Int8RotLinear(in, out, group)` for INT8 parts and by
    `LowRankLinear(in, out, rank)` for factorized parts; existing modules of those types are filled in place. Returns
    ``{"int8": [...], "lowrank": [...], "skipped": [...]}``: the model names filled, and the file's tensors that are
    not block linears (left to the caller).

    ``Int8RotLinear`` rotates its input by the block Hadamard of ``group``, so its weights must have been quantized
    in that rotated basis. Nothing in the reference tree says whether the ComfyUI release's INT8 weights were: the
    loader accepts INT8 parts only when the file's metadata names the group (``"convrot_group"``, which must equal
    ``group``) or the caller states it with ``rotated=True``; otherwise it raises ValueError instead of loading
    weights whose outputs would be silently wrong. Low-rank parts need neither."""
    from safetensors.torch import load_file

    info = check_metadata(path)
    declared = info.get(GROUP_KEY)
    if declared is not None and int(declared) != group:
        raise ValueError(f"{path}: INT8 weights quantized for Hadamard group {declared}, loader asked for {group}")
    basis_known = rotated or declared is not None
    parts, others = group_parts(load_file(path, device="cpu"))
    done: dict[str, list[str]] = {"int8": [], "lowrank": [], "skipped": sorted(others)}
    for (block, part), leaves in sorted(parts.items()):
        name = f"{prefix}.{block}.{MODULE_NAMES[part]}"
        target = _module(model, name)
        gated = part == "mlp.fc1"
        if "down.weight" in leaves or "up.weight" in leaves:
            down, up = leaves["down.weight"], leaves["up.weight"]
            if gated:
                up = _swap_halves(up)
            if not isinstance(target, LowRankLinear):
                target = replace_linear(model, name, LowRankLinear, down.shape[0])
            if tuple(down.shape) != tuple(target.down.weight.shape) or tuple(up.shape) != tuple(target.up.weight.shape):
                raise ValueError(f"{name}: factor shapes {tuple(down.shape)}, {tuple(up.shape)} do not match the model")
            target.down.weight.copy_(down.to(target.down.weight.dtype))
            target.up.weight.copy_(up.to(target.up.weight.dtype))
            done["lowrank"].append(name)
            continue
        if not basis_known:
            raise ValueError(f"{name}: the file does not say that its INT8 weights are in the block-Hadamard basis of "
                             f"group {group} (no {GROUP_KEY!r} metadata); pass rotated=True if they are")
        weight, scale = leaves["weight"], leaves["weight_scale"]
        if weight.dtype != torch.int8:
            raise ValueError(f"{name}: INT8 weight stored as {weight.dtype}")
        if "comfy_quant" in leaves:
            quant = decode_comfy_quant(leaves["comfy_quant"])
            if quant.get("format") != INT8_FORMAT:
                raise ValueError(f"{name}: comfy_quant format {quant.get('format')!r}, expected {INT8_FORMAT!r}")
        else:
            quant = {}
        n = weight.shape[0]
        scale = scale.to(torch.float32).flatten()
        if scale.numel() == 1:
            scale = scale.expand(n).clone()
        if scale.numel() != n:
            raise ValueError(f"{name}: weight_scale has {scale.numel()} values for {n} output channels")
        if gated:
            weight, scale = _swap_halves(weight), _swap_halves(scale)
        if not isinstance(target, Int8RotLinear):
            target = replace_linear(model, name, Int8RotLinear, group)
        if tuple(weight.shape) != tuple(target.qweight.shape):
            raise ValueError(f"{name}: weight shape {tuple(weight.shape)} != model {tuple(target.qweight.shape)}")
        target.qweight.copy_(weight)
        target.wscale.copy_(scale)
        target.comfy_quant = quant
        done["int8"].append(name)
    return done


__all__ = ["GROUP_KEY", "INT8_FORMAT", "METADATA_KEY", "MODULE_NAMES", "PART", "SUPPORTED_FORMAT", "check_metadata",
           "decode_comfy_quant", "group_parts", "hyperflow_metadata", "load_comfy_checkpoint"]
