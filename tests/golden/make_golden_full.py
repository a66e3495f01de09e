"""Writes tests/golden/full/*.npz: the reference's own CPU path at two benchmark sizes, stored as digests.

Runs in the development container only (the reference tree is not on the GPU machines). The small fixtures of
``make_golden.py`` hold whole tensors; at the benchmark sizes (M=1024, K=N=3072; M=32768,
K=5120, N=15360, the headline workload) the outputs are too large to commit, so each fixture stores:

* the seed and generator options (the inputs are rebuilt by ``oracle.make_inputs`` anywhere, bit for bit);
* the reference's ``sx`` in full and SHA-256 digests of its ``xq`` (int8 codes) and ``y`` (bf16 bits);
* every position where the reference differs from the exact-sum definition (the oracle): flat index, the
  reference's value and the oracle's value, for ``xr``, ``sx``, ``xq`` and ``y``;
* a sample of the reference's output rows, for a CPU check of the oracle that does not rebuild every row.

So a device output equal to the oracle everywhere becomes the reference's output once the listed positions are set
to the reference's values, which the digests confirm over every element (``tests/test_gpu_full_reference.py``).
Also the FFN down projection (M=32768, K=13824, N=5120) and a 41344-token block (M=41344) at the QKV width.

The reference path is ``Int8RotLinear.forward`` on CPU tensors (``_forward_torch``, int8.py:173-179), loaded from
``src/hyperflow_h3_flash/int8.py`` by file path as in ``make_golden.py``. The oracle's rows are computed for every
row (rotation and quantization) and, for the output, on the rows whose codes or scale differ plus a sample.
``python tests/golden/make_golden_full.py [name ...]``.
"""

from __future__ import annotations

import hashlib
import os
import platform
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

from oracle import oracle as O  # noqa: E402
from make_golden import Recorder, bits, from_bits, load_reference  # noqa: E402

#: name, (M, K, N, G), generator options (the 1024-token layer's and the QKV projection's distributions; the Hadamard group is 256 because
#: order 128 has no regular Hadamard matrix and the reference raises for it).
FULL = [
    ("full_cfg1", (1024, 3072, 3072, 256), dict(outlier_frac=0.01, outlier_scale=20.0, seed=21)),
    ("full_cfg2", (32768, 5120, 15360, 256), dict(outlier_frac=0.005, outlier_scale=30.0, seed=22)),
    # the FFN down projection (deep K) and a 41344-token block (40320 video + 1024 audio) at the QKV width
    ("full_cfg3_down", (32768, 13824, 5120, 256), dict(outlier_frac=0.005, outlier_scale=30.0, seed=23)),
    ("full_cfg4_qkv", (41344, 5120, 15360, 256), dict(outlier_frac=0.005, outlier_scale=30.0, seed=24)),
]
SAMPLE_ROWS = 8


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def reference_forward(ref, inputs, shape):
    """xr (bf16 bits), sx, xq, y (bf16 bits) of the reference forward, taken from the recorded program order."""
    m, k, n, g = shape
    layer = ref.Int8RotLinear(k, n, g)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inputs["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inputs["wscale"]))
    x = from_bits(inputs["x"])
    ref._rotation(g, torch.device("cpu"))

    class Keep(Recorder):
        # Keep only the tensors the fixture needs (the full recording of a 32768-row forward is ~12 GB).
        def __torch_function__(self, func, types, args=(), kwargs=None):
            out = func(*args, **(kwargs or {}))
            name = getattr(func, "__name__", str(func))
            if isinstance(out, torch.Tensor) and name in ("float", "div", "__truediv__", "clamp"):
                self.events.append((name, out))
            return out

    rec = Keep()
    with torch.no_grad(), rec:
        y = layer(x)
    xr = next(t for nm, t in rec.events if nm == "float" and t.shape == (m, k))
    sx = next(t for nm, t in rec.events if nm in ("div", "__truediv__") and t.shape == (m, 1)).reshape(-1)
    xq = next(t for nm, t in rec.events if nm == "clamp" and t.shape == (m, k))
    assert torch.equal(xq, xq.round())
    return bits(xr.to(torch.bfloat16)), sx.numpy().astype(np.float32), xq.numpy().astype(np.int8), bits(y)


def diff(ref: np.ndarray, orc: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    r, o = ref.reshape(-1), orc.reshape(-1)
    idx = np.flatnonzero(r != o)
    return idx.astype(np.int64), r[idx], o[idx]


def main():
    torch.manual_seed(0)
    ref = load_reference()
    meta = f"torch={torch.__version__} cpu={platform.processor() or platform.machine()} threads={torch.get_num_threads()}"
    rng = np.random.default_rng(2024)
    only = set(sys.argv[1:])  # fixture names to (re)write; all of them when none is given
    for name, shape, opts in FULL:
        if only and name not in only:
            continue
        m, k, n, g = shape
        t0 = time.time()
        inputs = O.make_inputs(m, k, n, g, **opts)
        xr_r, sx_r, xq_r, y_r = reference_forward(ref, inputs, shape)
        t1 = time.time()
        xr_o = O.rotate(inputs["x"], g)
        sx_o, xq_o = O.quantize(xr_o)
        t2 = time.time()
        out = {}
        for key, (a, b) in {"xr": (xr_r, xr_o), "sx": (sx_r, sx_o), "xq": (xq_r, xq_o)}.items():
            out[f"{key}_idx"], out[f"{key}_ref"], out[f"{key}_oracle"] = diff(a, b)
        # The oracle's output on every row whose codes or scale differ, plus a sample of the others; the remaining
        # rows have the same codes and scales, so their outputs are the same function of the same integers.
        moved = np.union1d(out["xq_idx"] // k, out["sx_idx"]).astype(np.int64)
        sample = np.sort(rng.choice(np.setdiff1d(np.arange(m), moved), size=SAMPLE_ROWS, replace=False))
        rows = np.union1d(moved, sample).astype(np.int64)
        y_o_rows = O.epilogue(O.int8_gemm(xq_o[rows], inputs["qweight"]), sx_o[rows], inputs["wscale"])
        y_diff = [(r * n + c, y_r[r, c], y_o_rows[i, c]) for i, r in enumerate(rows)
                  for c in np.flatnonzero(y_r[r] != y_o_rows[i])]
        out["y_idx"] = np.array([d[0] for d in y_diff], dtype=np.int64)
        out["y_ref"] = np.array([d[1] for d in y_diff], dtype=np.uint16)
        out["y_oracle"] = np.array([d[2] for d in y_diff], dtype=np.uint16)
        t3 = time.time()
        os.makedirs(os.path.join(HERE, "full"), exist_ok=True)
        path = os.path.join(HERE, "full", f"{name}.npz")
        np.savez_compressed(
            path, shape=np.array(shape, dtype=np.int64), meta=np.array(meta),
            opts=np.array(repr(sorted(opts.items()))), seed=np.array(opts["seed"]),
            outlier_frac=np.array(opts["outlier_frac"]), outlier_scale=np.array(opts["outlier_scale"]),
            sx=sx_r, xq_sha256=np.array(sha256(xq_r)), y_sha256=np.array(sha256(y_r)),
            sample_rows=sample.astype(np.int64), y_sample=y_r[sample], **out)
        print(f"{name}: M={m} K={k} N={n} G={g}: reference {t1 - t0:.1f} s, oracle {t2 - t1:.1f} s + {t3 - t2:.1f} s; "
              f"differ from the oracle: xr {out['xr_idx'].size}, sx {out['sx_idx'].size}, "
              f"xq {out['xq_idx'].size}, y {out['y_idx'].size} (rows {moved.size}) -> "
              f"{os.path.getsize(path) / 1024:.0f} KiB", flush=True)


if __name__ == "__main__":
    main()
