"""Writes the golden fixtures in tests/golden/*.npz from the reference's own CPU path.

Runs in the development container only (the reference tree is not on the GPU machines): it loads
``src/hyperflow_h3_flash/int8.py`` by file path (the package ``__init__`` imports diffusers, which is absent; int8.py
itself imports only torch), builds the reference ``Int8RotLinear``, and calls its ``forward`` on CPU tensors, which
takes the ``_forward_torch`` branch (int8.py:161-179). A ``TorchFunctionMode`` records every tensor the forward
produces, from which the intermediates are taken in program order:

* ``xr``  — the ``.float()`` of the bf16 rotation (int8.py:176);
* ``sx``  — the first ``div`` (int8.py:177);
* ``xq``  — the ``clamp`` (int8.py:178);
* ``acc`` — the second ``matmul`` (int8.py:179);
* ``y``   — the forward's output.

The composition fixture adds the low-rank branch ``up(down(x))`` of LowRankLinear (transformer.py:57-58; that file
imports diffusers, so it is restated here with two bias-free ``nn.Linear`` in bf16) and a bias, summed as separate
bf16 tensors the way three modules would compose.

Inputs come from the oracle's seeded generator, so the fixtures can be regenerated bit for bit:
``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import importlib.util
import os
import platform
import sys

import numpy as np
import torch
from torch.overrides import TorchFunctionMode

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

REFERENCE_INT8 = "/root/reference/src/hyperflow_h3_flash/int8.py"

#: name, (M, K, N, G), generator options. Shapes follow the fixture plan for this path: a slice of the 1024-token K=N=3072 layer,
#: the reference test's own (35, 128, 96, G=16), the kernel threshold M=17 at G=64, a single row, an odd M tail,
#: a slice of the M=32768 QKV projection, and one composition case with a rank-32 low-rank branch and a bias.
FIXTURES = [
    ("cfg1_slice", (64, 3072, 256, 256), dict(outlier_frac=0.01, outlier_scale=20.0, seed=11)),
    ("ref_test_shape", (35, 128, 96, 16), dict(outlier_frac=0.0, seed=12, weight_dist="quantized")),
    ("threshold_rows", (17, 512, 128, 64), dict(outlier_frac=0.01, outlier_scale=20.0, seed=13)),
    ("single_row", (1, 256, 64, 256), dict(outlier_frac=0.01, outlier_scale=20.0, seed=14)),
    ("odd_tail", (300, 1024, 128, 256), dict(outlier_frac=0.01, outlier_scale=30.0, seed=15,
                                             weight_dist="quantized")),
    ("cfg2_slice", (48, 5120, 64, 256), dict(outlier_frac=0.005, outlier_scale=30.0, seed=16)),
    ("composition", (64, 1024, 256, 256), dict(outlier_frac=0.01, outlier_scale=20.0, seed=17, rank=32,
                                               bias=True)),
]


def load_reference():
    spec = importlib.util.spec_from_file_location("reference_int8", REFERENCE_INT8)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


class Recorder(TorchFunctionMode):
    def __init__(self):
        super().__init__()
        self.events: list[tuple[str, object]] = []

    def __torch_function__(self, func, types, args=(), kwargs=None):
        out = func(*args, **(kwargs or {}))
        name = getattr(func, "__name__", str(func))
        if isinstance(out, torch.Tensor):
            self.events.append((name, out.detach().clone()))
        return out


def bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def run_reference(ref, inputs, shape):
    m, k, n, g = shape
    layer = ref.Int8RotLinear(k, n, g)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inputs["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inputs["wscale"]))
    x = from_bits(inputs["x"])
    ref._rotation(g, torch.device("cpu"))  # build the cached Hadamard outside the recorded forward
    rec = Recorder()
    with torch.no_grad(), rec:
        y = layer(x)
    names = [e[0] for e in rec.events]
    matmuls = [i for i, nm in enumerate(names) if nm in ("matmul", "__matmul__")]
    xr_i = next(i for i in range(matmuls[0], len(names)) if names[i] == "float")
    divs = [i for i, nm in enumerate(names) if nm in ("div", "__truediv__") and rec.events[i][1].shape == (m, 1)]
    clamp_i = next(i for i, nm in enumerate(names) if nm == "clamp" and rec.events[i][1].shape == (m, k))
    xr = rec.events[xr_i][1]
    sx = rec.events[divs[0]][1].reshape(-1)
    xq = rec.events[clamp_i][1]
    acc = rec.events[matmuls[1]][1]
    assert torch.equal(xq, xq.round()) and torch.equal(acc, acc.round()), "integer-valued intermediates"
    out = {
        "xr": bits(xr.to(torch.bfloat16)),
        "sx": sx.numpy().astype(np.float32),
        "xq": xq.numpy().astype(np.int8),
        "acc": acc.numpy().astype(np.int64).astype(np.int32),
        "y": bits(y),
    }
    assert torch.equal(xr.to(torch.bfloat16).float(), xr), "rotation is bf16-rounded"
    return out, y


def composition(inputs, y_int8):
    down = torch.nn.Linear(inputs["x"].shape[1], inputs["down"].shape[0], bias=False).to(torch.bfloat16)
    up = torch.nn.Linear(inputs["down"].shape[0], inputs["up"].shape[0], bias=False).to(torch.bfloat16)
    with torch.no_grad():
        down.weight.copy_(from_bits(inputs["down"]))
        up.weight.copy_(from_bits(inputs["up"]))
        x = from_bits(inputs["x"])
        u = down(x)
        lowrank = up(u)
        y = y_int8 + lowrank + from_bits(inputs["bias"])
    return {"u": bits(u), "lowrank": bits(lowrank), "y_composed": bits(y)}


def main():
    torch.manual_seed(0)
    ref = load_reference()
    meta = f"torch={torch.__version__} cpu={platform.processor() or platform.machine()} threads={torch.get_num_threads()}"
    for name, shape, opts in FIXTURES:
        m, k, n, g = shape
        opts = dict(opts)
        rank = opts.pop("rank", 0)
        bias = opts.pop("bias", False)
        inputs = O.make_inputs(m, k, n, g, rank=rank, bias=bias, **opts)
        out, y = run_reference(ref, inputs, shape)
        if rank:
            out.update(composition(inputs, y))
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, shape=np.array(shape, dtype=np.int64), meta=np.array(meta), **inputs, **out)
        print(f"{name}: M={m} K={k} N={n} G={g} -> {os.path.getsize(path) / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
