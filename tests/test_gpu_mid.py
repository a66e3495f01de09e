"""The 256 x 128 tile GEMM for a few hundred to a few thousand rows (mid_gemm_kernel) against the oracle.

The shapes below are ones the host sends to that kernel on a 256-CU device (its 256 x 256 tiles are fewer than the
CUs, the rows are too many for the skinny kernel, and its 256 x 128 tiles fill at least half the CUs; the test checks
the rule on the device's CU count). Bars as everywhere: without a low-rank branch or bias the bf16 outputs are
bitwise the oracle's (the reference's torch path); with them, within one bf16 ulp of the fused definition and 1e-2
of the reference composition; the fused tanh-GELU against the oracle's GELU of the unfused output (the bar of
test_gpu_activation.py). Ragged M and N, K not a multiple of the 128-byte stage, and K loops of two and three stages
(where the low-rank operands are loaded before or at the first boundary) are included. Rows are sampled for the
oracle; properties are checked on every row.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_utils import within_fp32_sum_bound

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def takes_band_path(m: int, n: int, r: int) -> bool:
    """The host's rule for the 128-row band tiles (band_blocks_n) on this device: one round of them fills at least
    7/8 of the CUs while the 256 x 128 tiles would fill at most 3/4."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    mid_tiles = -(-m // 256) * -(-n // 128)
    if r > 64 or (4 * mid_tiles > 3 * cus and mid_tiles <= cus):
        return False
    return any(cus >= -(-m // 128) * -(-n // (32 * nb)) and 8 * -(-m // 128) * -(-n // (32 * nb)) >= 7 * cus
               for nb in (5, 4, 3))


def takes_mid_path(m: int, n: int, r: int = 0) -> bool:
    """The host's rule (use_mid_gemm, after the band tiles' rule) on this device."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if takes_band_path(m, n, r):
        return False
    tiles_m = -(-m // 256)
    if tiles_m * -(-n // 256) >= cus:
        return False
    if m <= 128 or (m <= 256 and 2 * -(-n // 128) <= cus):
        return False
    return 2 * tiles_m * -(-n // 128) >= cus


CASES = [
    # m, k, n, group, rank, bias
    (1024, 5120, 7168, 256, 0, False),
    (1024, 5120, 7168, 256, 32, False),
    (256, 5120, 30720, 256, 32, False),
    (700, 5136, 8000, 16, 0, False),
    (700, 5136, 8000, 16, 24, True),
    (300, 256, 16384, 256, 0, False),
    (300, 256, 16384, 256, 64, True),
    (520, 384, 8192, 64, 16, False),
    (1500, 2048, 4000, 256, 64, True),
]


def layer_for(m, k, n, g, r, bias, seed, activation=None):
    from hyperflow_h3_flash_amd import Int8RotLinear

    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k, device=DEV, generator=gen)
    cols = torch.randperm(k, device=DEV, generator=gen)[: max(1, k // 200)]
    x[:, cols] *= 30.0
    x = x.to(torch.bfloat16)
    layer = Int8RotLinear(k, n, g, rank=r, bias=bias, activation=activation).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen))
        layer.wscale.copy_(torch.rand(n, device=DEV, generator=gen) * 9e-3 + 1e-3)
        if r:
            layer.down.weight.copy_((torch.randn(r, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16))
            layer.up.weight.copy_((torch.randn(n, r, device=DEV, generator=gen) * 0.02).to(torch.bfloat16))
        if bias:
            layer.bias.copy_((torch.randn(n, device=DEV, generator=gen) * 0.01).to(torch.bfloat16))
    return x, layer


def sampled(m, seed, count=16):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([rng.choice(m, size=min(count, m), replace=False), [0, 255 % m],
                                     np.arange(max(0, m - 3), m)]))


@pytest.mark.parametrize("m,k,n,g,r,bias", CASES)
def test_mid_tiles_match_the_oracle(oracle_lib, m, k, n, g, r, bias):
    assert takes_mid_path(m, n, r), "this shape should take the 256 x 128 tile kernel"
    x, layer = layer_for(m, k, n, g, r, bias, seed=m + n + r)
    with torch.no_grad():
        y = layer(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y.float()).all())
    rows = sampled(m, m + k)
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
    if r:
        from hyperflow_h3_flash_amd.int8 import lowrank_down

        u_dev = lowrank_down(x[torch.from_numpy(rows).to(DEV)], layer.down.weight)
        assert within_fp32_sum_bound(oracle_lib.bf16_to_f32(bits_of(u_dev)), oracle_lib.bf16_to_f32(u_ref),
                                     oracle_lib.bf16_to_f32(xb), oracle_lib.bf16_to_f32(down))
    fused = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(out["acc"], out["sx"], ws, u_ref, up, b))
    g32 = oracle_lib.bf16_to_f32(got)
    assert (np.abs(g32 - fused) <= np.abs(fused) * 2.0**-7 + 1e-6).all()
    comp = oracle_lib.bf16_to_f32(oracle_lib.composition(out["y"], xb, down, up, b))
    assert np.abs(g32 - comp).max() / np.abs(comp).max() <= 1e-2


@pytest.mark.parametrize("m,k,n,r", [(1024, 5120, 7168, 64), (700, 2048, 8000, 0)])
def test_mid_tiles_gelu_epilogue(oracle_lib, m, k, n, r):
    assert takes_mid_path(m, n, r)
    x, layer = layer_for(m, k, n, 256, r, False, seed=7 + m, activation="gelu_tanh")
    with torch.no_grad():
        h = layer(x)
        layer.activation = None
        pre = layer(x)
    torch.cuda.synchronize()
    rows = sampled(m, 11)
    pre_bits = bits_of(pre[rows])
    got = oracle_lib.bf16_to_f32(bits_of(h[rows]))
    ref = oracle_lib.bf16_to_f32(oracle_lib.gelu_tanh(pre_bits))
    assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()
    region = oracle_lib.bf16_to_f32(pre_bits) >= -3.0
    assert (got[region] == ref[region]).mean() >= 0.999


def test_mid_tiles_agree_with_the_persistent_tiles_bitwise():
    """The same layer (with a bias) through the 256 x 128 tiles and, as part of a 4096-row batch, through the
    persistent 256 x 256 tiles: rows are computed independently by the same arithmetic, so they agree bit for bit."""
    x, layer = layer_for(1024, 5120, 7168, 256, 0, True, seed=3)
    assert takes_mid_path(1024, 7168)
    big = torch.cat([x, x, x, x], dim=0)  # 4096 rows: 256 x 256 tiles fill the CUs, no mid path
    assert not takes_mid_path(4096, 7168)
    with torch.no_grad():
        y_mid = layer(x)
        y_big = layer(big)
    torch.cuda.synchronize()
    assert torch.equal(y_mid.view(torch.int16), y_big[:1024].view(torch.int16))
