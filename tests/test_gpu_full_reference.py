"""The device path against the reference's own CPU path at four benchmark sizes, every element (GPU).

tests/golden/full/*.npz hold the reference ``Int8RotLinear.forward`` on CPU tensors (int8.py:161-179) at M=1024,
K=N=3072, at the headline shape M=32768, K=5120, N=15360, at the FFN down projection M=32768, K=13824,
N=5120 and at the 41344-token block's QKV width M=41344, K=5120, N=15360 (G=256, no low-rank branch, no bias) as SHA-256 digests
of its codes and outputs, its scales in full, and the list of positions where it differs from the exact-sum
definition (each explained by its fp32 accumulation; test_full_reference.py). Inputs are rebuilt from the seed.

Bars: the device's scales equal the reference's bit for bit; the device's codes and outputs hold the oracle's values
at every listed position and, with those positions set to the reference's values, hash to the reference's digests —
so they equal the reference's output on every other element.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from full_reference import FULL_FIXTURES, inputs, load, patched_digest

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


@pytest.mark.parametrize("name", FULL_FIXTURES)
def test_device_equals_reference_at_full_size(name):
    from hyperflow_h3_flash_amd import Int8RotLinear
    from hyperflow_h3_flash_amd.int8 import _kernels

    fx = load(name)
    m, k, n, g = (int(v) for v in fx["shape"])
    print(f"full-size reference check {name}: M={m} K={k} N={n} G={g}", flush=True)
    inp = inputs(fx)
    x = torch.from_numpy(inp["x"].view(np.int16)).view(torch.bfloat16).to(DEV)
    layer = Int8RotLinear(k, n, g).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        xq, sx = _kernels().rotate_quant(x, g)
        y = layer(x)
    torch.cuda.synchronize()
    sx_h = sx.reshape(-1).cpu().numpy()
    assert np.array_equal(sx_h.view(np.uint32), fx["sx"].view(np.uint32))
    xq_h = xq.cpu().numpy()
    assert np.array_equal(xq_h.reshape(-1)[fx["xq_idx"]], fx["xq_oracle"])
    assert patched_digest(xq_h, fx["xq_idx"], fx["xq_ref"]) == str(fx["xq_sha256"])
    del xq
    y_h = y.cpu().view(torch.int16).numpy().view(np.uint16)
    del y
    assert np.array_equal(y_h.reshape(-1)[fx["y_idx"]], fx["y_oracle"])
    assert patched_digest(y_h, fx["y_idx"], fx["y_ref"]) == str(fx["y_sha256"])
