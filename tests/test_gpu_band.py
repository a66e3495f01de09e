"""The 128-row band tile GEMM (band_gemm_kernel: 128 x 32 NB tiles, NB = 3, 4 or 5) against the oracle.

The shapes below are ones the host sends to that kernel on a 256-CU device: one round of 128-row tiles fills at least
7/8 of the CUs while the 256 x 128 tiles would fill at most 3/4 (the test checks the rule on the device's CU count).
Bars as for the other tile kernels: without a low-rank branch or bias the bf16 outputs are bitwise the oracle's (the
reference's torch path); with them, within one bf16 ulp (2^-7 relative) of the fused definition and 1e-2 of the
reference composition; the fused tanh-GELU against the oracle's GELU of the unfused output. Included: the single
layer of 1024 tokens (M=1024, K=N=3072, rank 32, bias; 128 x 96 tiles), M=1024 with N=4096 and 5120 (128 x 128, 128 x 160), 768
rows (128 x 128: six tile rows), ragged M and N with K not a multiple of the 128-byte stage, and K loops of two and
three stages (the low-rank operands loaded with the first stages). The rows are computed independently, so the same
rows through the persistent 256 x 256 tiles (as part of a 4096-row batch) agree bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_mid import bits_of, layer_for, sampled, takes_band_path

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


CASES = [
    # m, k, n, group, rank, bias
    (1024, 3072, 3072, 256, 32, True),
    (1024, 3072, 3072, 256, 0, False),
    (1024, 4096, 4096, 256, 64, False),
    (1024, 5120, 5120, 256, 0, False),
    (1024, 5120, 5120, 256, 32, True),
    (768, 5120, 5120, 256, 32, False),
    (700, 5136, 6000, 16, 0, False),
    (700, 5136, 6000, 16, 24, True),
    (1000, 256, 5000, 256, 64, True),
    (1024, 384, 5120, 64, 32, False),
]


@pytest.mark.parametrize("m,k,n,g,r,bias", CASES)
def test_band_tiles_match_the_oracle(oracle_lib, m, k, n, g, r, bias):
    assert takes_band_path(m, n, r), "this shape should take the 128-row band tiles"
    print(f"band tiles M={m} K={k} N={n} G={g} r={r} bias={bias}", flush=True)
    x, layer = layer_for(m, k, n, g, r, bias, seed=m + n + r + 1)
    with torch.no_grad():
        y = layer(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y.float()).all())
    rows = sampled(m, m + k + 1)
    xb = bits_of(x[rows])
    w, ws = layer.qweight.cpu().numpy(), layer.wscale.cpu().numpy()
    out = oracle_lib.convrot_linear(xb, w, ws, g)
    got = bits_of(y[rows])
    if not r and not bias:
        np.testing.assert_array_equal(got, out["y"])
        return
    down = bits_of(layer.down.weight) if r else None
    up = bits_of(layer.up.weight) if r else None
    b = bits_of(layer.bias) if bias else None
    u_ref = oracle_lib.lowrank_down(xb, down) if r else None
    fused = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(out["acc"], out["sx"], ws, u_ref, up, b))
    g32 = oracle_lib.bf16_to_f32(got)
    assert (np.abs(g32 - fused) <= np.abs(fused) * 2.0**-7 + 1e-6).all()
    comp = oracle_lib.bf16_to_f32(oracle_lib.composition(out["y"], xb, down, up, b))
    assert np.abs(g32 - comp).max() / np.abs(comp).max() <= 1e-2


@pytest.mark.parametrize("m,k,n,r", [(1024, 5120, 5120, 64), (1024, 3072, 3072, 0)])
def test_band_tiles_gelu_epilogue(oracle_lib, m, k, n, r):
    assert takes_band_path(m, n, r)
    print(f"band tiles GELU M={m} K={k} N={n} r={r}", flush=True)
    x, layer = layer_for(m, k, n, 256, r, False, seed=13 + m, activation="gelu_tanh")
    with torch.no_grad():
        h = layer(x)
        layer.activation = None
        pre = layer(x)
    torch.cuda.synchronize()
    rows = sampled(m, 17)
    pre_bits = bits_of(pre[rows])
    got = oracle_lib.bf16_to_f32(bits_of(h[rows]))
    ref = oracle_lib.bf16_to_f32(oracle_lib.gelu_tanh(pre_bits))
    assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()
    region = oracle_lib.bf16_to_f32(pre_bits) >= -3.0
    assert (got[region] == ref[region]).mean() >= 0.999


@pytest.mark.parametrize("m,k,n,r,bias", [(1024, 5120, 5120, 0, True), (700, 5136, 6000, 0, True)])
def test_band_tiles_agree_with_the_persistent_tiles_bitwise(m, k, n, r, bias):
    """The same rows through the band tiles and, as part of a 4096-row batch, through the persistent 256 x 256 tiles
    (a different tile, K loop and epilogue code, the same arithmetic): bitwise equal, bias included. (Rank 0: the
    low-rank intermediate itself is summed in another order at 1024 rows, where its projection splits K, than at
    4096.)"""
    x, layer = layer_for(m, k, n, 256 if k % 256 == 0 else 16, r, bias, seed=5 + m)
    assert takes_band_path(m, n, r)
    big = torch.cat([x, x, x, x, x, x][: -(-4096 // m)], dim=0)
    assert not takes_band_path(big.shape[0], n, r)
    with torch.no_grad():
        y_band = layer(x)
        y_big = layer(big)
    torch.cuda.synchronize()
    assert torch.equal(y_band.view(torch.int16), y_big[:m].view(torch.int16))
