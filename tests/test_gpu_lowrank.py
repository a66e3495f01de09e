"""The standalone low-rank linear and the fused Q/K/V projection on the gfx950 kernels.

Bars: the low-rank branch within one bf16 ulp of the oracle's exactly rounded sums (the device sums in fp32, the
oracle in float64) and bitwise on almost every element; zero-padded ranks and the fused Q/K/V projection bitwise
equal to the unpadded / separate layers.
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


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def within_one_ulp(got_bits, ref_bits, lib):
    got, ref = lib.bf16_to_f32(got_bits), lib.bf16_to_f32(ref_bits)
    return (np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 1e-30).all(), (got == ref).mean()


@pytest.mark.parametrize("m,n,r,bias", [(1, 8, 8, False), (100, 200, 64, True), (300, 520, 136, False),
                                        (257, 1000, 200, True), (128, 128, 8, False)])
def test_lowrank_up_matches_oracle(oracle_lib, m, n, r, bias):
    from hyperflow_h3_flash_amd.int8 import lowrank_up

    rng = np.random.default_rng(m + n + r)
    u = oracle_lib.f32_to_bf16(rng.standard_normal((m, r)).astype(np.float32))
    up = oracle_lib.f32_to_bf16((rng.standard_normal((n, r)) * 0.02).astype(np.float32))
    b = oracle_lib.f32_to_bf16((rng.standard_normal(n) * 0.01).astype(np.float32)) if bias else None
    y = lowrank_up(to_dev_bf16(u), to_dev_bf16(up), None if b is None else to_dev_bf16(b))
    ok, exact = within_one_ulp(bits_of(y), oracle_lib.lowrank_up(u, up, b), oracle_lib)
    assert ok and exact > 0.98


@pytest.mark.parametrize("m,n,r,bias", [(4096, 4096, 256, False), (4100, 4200, 136, True), (2048, 8448, 512, True),
                                        (4096, 4096, 128, False)])
def test_lowrank_up_on_the_persistent_tiles_matches_oracle(oracle_lib, m, n, r, bias):
    """Ranks from 128 with at least one round of 256 x 256 output tiles take the persistent tile kernel's bf16
    product (r=136: a K of 272 bytes, a partial last stage; r=128: two stages): sampled rows
    (the first, the last and ragged tile edges included) within the error bound of an fp32 sum of the rank's products
    of the oracle's exactly rounded sum, bitwise on almost every element, every row finite."""
    from hyperflow_h3_flash_amd.int8 import lowrank_up

    assert ((m + 255) // 256) * ((n + 255) // 256) >= 256  # the tile route at 256 CUs
    gen = torch.Generator(device=DEV).manual_seed(m + n + r)
    u = (torch.randn(m, r, device=DEV, generator=gen)).to(torch.bfloat16)
    up = (torch.randn(n, r, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, device=DEV, generator=gen) * 0.01).to(torch.bfloat16) if bias else None
    print(f"lowrank_up tiles M={m} N={n} r={r} bias={bias}", flush=True)
    y = lowrank_up(u, up, b)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y.float()).all())
    rows = np.unique(np.concatenate([[0, 255, 256], np.arange(m - 3, m),
                                     np.random.default_rng(m).choice(m, size=12, replace=False)]))
    u_rows = bits_of(u[torch.from_numpy(rows).to(DEV)])
    want = oracle_lib.lowrank_up(u_rows, bits_of(up), None if b is None else bits_of(b))
    got = oracle_lib.bf16_to_f32(bits_of(y[torch.from_numpy(rows).to(DEV)]))
    ref = oracle_lib.bf16_to_f32(want)
    # an fp32 sum of r products in any order, rounded once (a bias, when present, is one more exact term)
    assert within_fp32_sum_bound(got, ref, oracle_lib.bf16_to_f32(u_rows), oracle_lib.bf16_to_f32(bits_of(up)))
    assert (got == ref).mean() > 0.98


def test_lowrank_linear_matches_the_reference_composition(oracle_lib):
    """`LowRankLinear(x) = up(down(x))` against the reference modules' own output (the composition fixture)."""
    from golden_utils import load_fixture

    from hyperflow_h3_flash_amd import LowRankLinear

    f = load_fixture("composition")
    k, r, n = f["x"].shape[1], f["down"].shape[0], f["up"].shape[0]
    layer = LowRankLinear(k, n, r).to(DEV, torch.bfloat16)
    with torch.no_grad():
        layer.down.weight.copy_(to_dev_bf16(f["down"]))
        layer.up.weight.copy_(to_dev_bf16(f["up"]))
        y = layer(to_dev_bf16(f["x"]))
    ok, exact = within_one_ulp(bits_of(y), f["lowrank"], oracle_lib)
    assert ok and exact > 0.98
    # and against the oracle's chain on the same inputs
    ref = oracle_lib.lowrank_up(oracle_lib.lowrank_down(f["x"], f["down"]), f["up"])
    ok, exact = within_one_ulp(bits_of(y), ref, oracle_lib)
    assert ok and exact > 0.98


def test_rank_padding_is_bitwise_neutral():
    """Zero rows of down and columns of up add exact zeros: padded and trimmed layers agree bit for bit."""
    from hyperflow_h3_flash_amd import LowRankLinear, set_lowrank_rank_multiple

    torch.manual_seed(0)
    layer = LowRankLinear(512, 384, 40).to(DEV, torch.bfloat16)
    with torch.no_grad():
        layer.down.weight.mul_(0.05)
        layer.up.weight.mul_(0.05)
    x = torch.randn(77, 512, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        base = layer(x)
        assert layer.pad_rank(64)
        padded = layer(x)
        holder = torch.nn.Sequential(layer)
        assert set_lowrank_rank_multiple(holder, 8) == 1 and layer.rank == 40
        trimmed = layer(x)
    assert torch.equal(base, padded) and torch.equal(base, trimmed)


@pytest.mark.parametrize("rank,bias", [(0, False), (32, True)])
def test_fused_qkv_is_bitwise_the_three_projections(oracle_lib, rank, bias):
    from hyperflow_h3_flash_amd import Int8RotLinear, fuse_qkv

    k, g, widths = 1024, 256, (256, 384, 128)
    rng = np.random.default_rng(rank)
    layers = []
    down = torch.randn(rank, k, device=DEV).mul_(0.02).to(torch.bfloat16) if rank else None
    for n in widths:
        layer = Int8RotLinear(k, n, g, rank=rank, bias=bias).to(DEV)
        with torch.no_grad():
            layer.qweight.copy_(torch.from_numpy(rng.integers(-127, 128, size=(n, k)).astype(np.int8)))
            layer.wscale.copy_(torch.from_numpy(rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)))
            if rank:
                layer.down.weight.copy_(down)
                layer.up.weight.copy_(torch.randn(n, rank, device=DEV).mul_(0.02))
            if bias:
                layer.bias.copy_(torch.randn(n, device=DEV).mul_(0.01))
        layers.append(layer)
    fused = fuse_qkv(*layers)
    x = to_dev_bf16(oracle_lib.make_inputs(300, k, 8, g, seed=rank)["x"])
    with torch.no_grad():
        separate = torch.cat([layer(x) for layer in layers], dim=-1)
        together = fused(x)
    assert torch.equal(separate, together)


def test_lowrank_linear_keeps_float32_and_float64_precision():
    """A float32 / float64 LowRankLinear on the device is the reference's ``up(down(x))`` in its own dtype (no
    rounding to bf16); only bf16 inputs take the HIP kernels."""
    from hyperflow_h3_flash_amd import LowRankLinear

    torch.manual_seed(5)
    for dtype in (torch.float32, torch.float64):
        layer = LowRankLinear(256, 96, 24).to(device=DEV, dtype=dtype)
        x = torch.randn(7, 3, 256, device=DEV, dtype=dtype)
        with torch.no_grad():
            y = layer(x)
            expected = layer.up(layer.down(x))
        assert y.dtype == dtype
        torch.testing.assert_close(y, expected, rtol=0, atol=0)


def test_device_layer_without_the_library_raises(monkeypatch):
    """With no HIP library the layers refuse device tensors (there is no device fallback)."""
    from hyperflow_h3_flash_amd import Int8RotLinear, LowRankLinear
    from hyperflow_h3_flash_amd import int8 as int8_mod
    from hyperflow_h3_flash_amd import lowrank as lowrank_mod

    monkeypatch.setattr(int8_mod, "_kernels", lambda: None)
    monkeypatch.setattr(lowrank_mod, "_kernels", lambda: None)
    layer = Int8RotLinear(256, 64, 256).to(DEV)
    with pytest.raises(RuntimeError, match="HIP library"):
        layer(torch.randn(4, 256, device=DEV, dtype=torch.bfloat16))
    lr = LowRankLinear(256, 64, 8).to(device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP library"):
        lr(torch.randn(4, 256, device=DEV, dtype=torch.bfloat16))


@pytest.mark.parametrize("m,k,r", [(16500, 1040, 72), (20000, 5376, 256), (17000, 2048, 200), (33000, 1024, 320),
                                   (33000, 1024, 512), (37710, 5376, 128), (37710, 5376, 256), (40000, 2064, 200),
                                   (37710, 5376, 200), (37710, 14336, 256), (37710, 5376, 512),
                                   (37710, 4112, 136), (36000, 4224, 264), (40960, 4288, 392)])
def test_wide_rank_down_projection(oracle_lib, m, k, r):
    """Ranks past 64 with more rows than half the CUs' 128-row workgroups cover (no K split) take 256 ranks per pass
    over x (lowrank_down_wide_kernel): the same sums, in the same order, as 64-rank passes of the unsplit rank-64
    kernel (bitwise). Against the exact sums s (float64, sampled rows): bitwise the oracle's exactly rounded value on
    almost every element, and everywhere within the fp32 accumulation bound, |u - s| <= 2^-8 |s| + (1 + 2^-8) K
    2^-24 sum_k |x_k d_k| (a sum that cancels to near zero can miss one bf16 ulp of itself). M=37710 with r=128 uses
    workgroups of five row blocks. From r=192 with enough 256-row blocks to fill half the CUs (M=33000, r=320 and
    512; M=40000, r=200 with a partial column tile and K=2064, not a multiple of the 64-element stage) the persistent
    tile kernel's bf16 product runs instead, and past r=128 with K >= 4096 and 160-row blocks filling 7/8 of the CUs
    (M=37710: r=200 with seven live rank blocks of eight, r=256, r=512 in two passes, K=5376 and 14336) the 8-wave
    kernel with the down slab staged through registers, all with the same summation order. Its last three cases end
    the stage loop on each of the three register buffers (65, 66 and 67 stages of 64 elements, the first with a
    partial last stage and a partial last row block), with 136, 264 and 392 ranks (passes whose last live wave holds
    only 8 of its 32 ranks)."""
    from hyperflow_h3_flash_amd import _native
    from hyperflow_h3_flash_amd.int8 import _stream, lowrank_down

    print(f"wide-rank low-rank down M={m} K={k} r={r}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(m + k + r)
    x = (torch.randn(m, k, device=DEV, generator=gen) * 2.0).to(torch.bfloat16)
    down = (torch.randn(r, k, device=DEV, generator=gen) * 0.05).to(torch.bfloat16)
    u = lowrank_down(x, down)
    lib = _native.library()
    ref = torch.empty(m, r, device=DEV, dtype=torch.bfloat16)
    for j0 in range(0, r, 64):
        rr = min(64, r - j0)
        assert lib.hf_lowrank_down(x.data_ptr(), k, down[j0:].data_ptr(), k, ref[:, j0:].data_ptr(), r, m, k, rr,
                                   _stream(DEV)) == 0
    torch.cuda.synchronize()
    assert torch.equal(u, ref)
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(r).choice(m, 24, replace=False)]))
    xs, ds = bits_of(x[rows]), bits_of(down)
    got = oracle_lib.bf16_to_f32(bits_of(u[rows])).astype(np.float64)
    xf, df = oracle_lib.bf16_to_f32(xs).astype(np.float64), oracle_lib.bf16_to_f32(ds).astype(np.float64)
    exact_sum, mag = xf @ df.T, np.abs(xf) @ np.abs(df).T
    assert (np.abs(got - exact_sum) <= 2.0**-8 * np.abs(exact_sum) + (1 + 2.0**-8) * k * 2.0**-24 * mag).all()
    assert (bits_of(u[rows]) == oracle_lib.lowrank_down(xs, ds)).mean() > 0.98


@pytest.mark.parametrize("m,k,r,px,pd,pu", [(37710, 4112, 136, 16, 24, 16), (37710, 5376, 256, 64, 8, 8),
                                            (33000, 1024, 320, 8, 8, 8)])
def test_wide_rank_down_projection_with_padded_strides(m, k, r, px, pd, pu):
    """The wide-rank routes (the 8-wave kernel at M=37710, the persistent tiles at M=33000) with x, down and u in
    padded rows: bitwise the result on contiguous copies, and u's padding columns untouched."""
    from hyperflow_h3_flash_amd import _native
    from hyperflow_h3_flash_amd.int8 import _stream

    lib = _native.library()
    print(f"padded wide-rank low-rank down M={m} K={k} r={r} pads {px} {pd} {pu}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(m + k + r)
    xs = (torch.randn(m, k + px, device=DEV, generator=gen) * 2.0).to(torch.bfloat16)
    ds = (torch.randn(r, k + pd, device=DEV, generator=gen) * 0.05).to(torch.bfloat16)
    us = torch.full((m, r + pu), -1.0, device=DEV, dtype=torch.bfloat16)
    x, d = xs[:, :k].contiguous(), ds[:, :k].contiguous()
    u = torch.empty(m, r, device=DEV, dtype=torch.bfloat16)
    nb = lib.hf_lowrank_down_ws_bytes(m, k, r)
    ws = torch.empty(max(nb, 1), device=DEV, dtype=torch.uint8)
    for xx, ldx, dd, ldd, uu, ldu in ((xs, k + px, ds, k + pd, us, r + pu), (x, k, d, k, u, r)):
        assert lib.hf_lowrank_down_ws(xx.data_ptr(), ldx, dd.data_ptr(), ldd, uu.data_ptr(), ldu, m, k, r,
                                      ws.data_ptr(), nb, _stream(DEV)) == 0
    torch.cuda.synchronize()
    assert torch.equal(us[:, :r], u)
    assert bool((us[:, r:] == -1.0).all())


@pytest.mark.parametrize("m,k,n,r", [(37710, 5376, 7168, 256), (37710, 14336, 5376, 512), (4096, 3072, 3072, 200)])
def test_lowrank_linear_matches_torch_on_the_device(m, k, n, r):
    """The standalone layer against what the reference runs for it on a GPU, torch's own bf16 `up(down(x))`
    (transformer.py:57-58; the vendor library's GEMMs), at the model's sizes: the intermediate u within the fp32
    accumulation bound of torch's and equal on >= 99.9 % of elements, the output equal on >= 99 % and within 1e-2 of
    its largest magnitude (measured: bitwise everywhere at K=5376, 99.75-99.98 % at the other two, where the
    vendor sums K in another order)."""
    from hyperflow_h3_flash_amd import LowRankLinear
    from hyperflow_h3_flash_amd.int8 import lowrank_down

    print(f"low-rank linear against torch M={m} K={k} N={n} r={r}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(m + k + r)
    layer = LowRankLinear(k, n, r).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        layer.down.weight.copy_(torch.randn(r, k, device=DEV, generator=gen) * 0.02)
        layer.up.weight.copy_(torch.randn(n, r, device=DEV, generator=gen) * 0.02)
        x = torch.randn(m, k, device=DEV, generator=gen).to(torch.bfloat16)
        y = layer(x)
        u = lowrank_down(x, layer.down.weight)
        u_t = layer.down(x)
        y_t = layer.up(u_t)
        mag = x.float().abs() @ layer.down.weight.float().abs().t().contiguous()
    torch.cuda.synchronize()
    du = (u.float() - u_t.float()).abs()
    assert bool((du <= 2.0**-7 * u_t.float().abs() + 2 * k * 2.0**-24 * mag).all())
    assert float((u.view(torch.int16) == u_t.view(torch.int16)).float().mean()) >= 0.999
    assert float((y.view(torch.int16) == y_t.view(torch.int16)).float().mean()) >= 0.99
    assert float((y.float() - y_t.float()).abs().max() / y_t.float().abs().max()) <= 1e-2
