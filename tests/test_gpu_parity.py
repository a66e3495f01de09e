"""Parity of the gfx950 HIP path with the oracle and with the reference's golden vectors.

Bars: bit-exact int8 codes, per-token scales, int32 accumulators and (no low-rank, no bias) bf16 outputs; the fused
low-rank + bias extension within 1e-2 of the reference composition, max |y - y_ref| / max |y_ref|.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from golden_utils import (check_against_composition, classify_rotation_mismatches, device_lowrank_slack, fixture_names,
                          load_fixture, within_fp32_sum_bound)

pytestmark = pytest.mark.gpu

FIXTURES = fixture_names()
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()  # fails loudly when the HIP library is missing


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make_layer(inp, k, n, g, **kw):
    from hyperflow_h3_flash_amd import Int8RotLinear

    layer = Int8RotLinear(k, n, g, **kw).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
    return layer


# ------------------------------------------------------------------------------------------------ GEMM accumulator


@pytest.mark.parametrize("m,n,k", [(1, 16, 16), (32, 32, 128), (256, 256, 128), (300, 200, 1040), (513, 257, 2064),
                                   (64, 1000, 5120)])
def test_gemm_i32_is_the_exact_integer_product(oracle_lib, m, n, k):
    from hyperflow_h3_flash_amd.int8 import int8_gemm_i32

    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, size=(n, k), dtype=np.int64).astype(np.int8)
    acc = int8_gemm_i32(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV))
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle_lib.int8_gemm(a, b))


def test_gemm_i32_extreme_codes(oracle_lib):
    from hyperflow_h3_flash_amd.int8 import int8_gemm_i32

    a = np.full((40, 14336), -127, dtype=np.int8)
    a[1::2] = 127
    b = np.full((48, 14336), 127, dtype=np.int8)
    acc = int8_gemm_i32(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV))
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle_lib.int8_gemm(a, b))


@pytest.mark.parametrize("m,n,k", [(32768, 15360, 5120), (37710, 5376, 14336)])
def test_gemm_i32_equals_the_vendor_int8_gemm_at_full_size(m, n, k):
    """The int32 accumulator at the headline shape and the model's down projection against the vendor library's
    INT8 GEMM (torch._int_mm, what the reference's cuBLASLt backend computes, int8.py:362): integer sums, so equal
    everywhere."""
    from hyperflow_h3_flash_amd.int8 import int8_gemm_i32

    print(f"int32 accumulator against torch._int_mm M={m} N={n} K={k}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(m + n + k)
    a = torch.randint(-127, 128, (m, k), device=DEV, dtype=torch.int8, generator=gen)
    b = torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen)
    acc = int8_gemm_i32(a, b)
    want = torch._int_mm(a, b.t())
    torch.cuda.synchronize()
    assert torch.equal(acc, want)


# -------------------------------------------------------------------------------------------- rotate + quantize


@pytest.mark.parametrize("name", FIXTURES)
def test_rotate_quant_matches_oracle_and_golden(oracle_lib, name):
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    f = load_fixture(name)
    q, s = rotate_quant(to_dev_bf16(f["x"]), f["G"])
    q, s = q.cpu().numpy(), s.cpu().numpy()
    xr = oracle_lib.rotate(f["x"], f["G"])
    sx, xq = oracle_lib.quantize(xr)
    np.testing.assert_array_equal(s, sx)
    np.testing.assert_array_equal(q, xq)
    # against the reference's own torch-CPU outputs: equal wherever its fp32-accumulated rotation is
    mism, unexplained = classify_rotation_mismatches(f["x"], xr, f["xr"], f["G"])
    assert not unexplained
    np.testing.assert_array_equal(s, f["sx"])
    np.testing.assert_array_equal(q, f["xq"])


@pytest.mark.parametrize("group", [4, 16, 64, 256])
@pytest.mark.parametrize("m,k", [(1, 256), (7, 1280), (65, 2304), (130, 5120)])
def test_rotate_quant_groups_and_partial_tiles(oracle_lib, group, m, k):
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    inp = oracle_lib.make_inputs(m, k, 16, group, outlier_frac=0.01, outlier_scale=30.0, seed=group + m + k)
    q, s = rotate_quant(to_dev_bf16(inp["x"]), group)
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(inp["x"], group))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)


@pytest.mark.parametrize("m,k", [(3, 14336), (3, 16384), (1025, 1024), (1024, 13824), (2, 77312), (1030, 5120),
                                 (1100, 5376), (1027, 13824), (1025, 20480), (1025, 21504), (1029, 7168),
                                 (1031, 14336)])
def test_rotate_quant_both_row_layouts(oracle_lib, m, k):
    """Up to 1024 rows of at most 14 tiles run one workgroup per row. More rows of up to 20 tiles keep the row in
    registers, split over 1 (<= 5 tiles), 2 (6: a partial last tile), 3 (14) or 4 (20) waves per row; wider rows
    run one wave per row with an LDS row buffer. All against the oracle, on either side of each threshold and at the
    widest supported row."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    inp = oracle_lib.make_inputs(m, k, 8, 256, outlier_frac=0.005, outlier_scale=30.0, seed=m + k)
    q, s = rotate_quant(to_dev_bf16(inp["x"]), 256)
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(inp["x"], 256))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)


@pytest.mark.parametrize("group", [4, 16, 64, 256])
def test_rotate_quant_rounds_exact_ties_to_even(oracle_lib, group):
    """Rotated sums that land exactly halfway between two bf16 values, and just beside halfway, at many binades
    (the once-only rounding of the exact sum, ties to even), in both row layouts."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    rng = np.random.default_rng(group)
    m, k = 1100, 1024
    x = np.zeros((m, k), dtype=np.float32)
    # per group of the row: one large value 2^e * (1 + j/128) and one small value at the half-unit 2^(e-8) (an exact
    # tie for every output of the group) or at 3 half-units (a tie on the other side), or one quarter-unit off
    e = rng.integers(-30, 30, size=(m, k // group)).astype(np.float64)
    big = np.exp2(e) * (1.0 + rng.integers(0, 128, size=e.shape) / 128.0) * rng.choice([-1.0, 1.0], size=e.shape)
    small = np.exp2(e - 8) * rng.choice([1.0, 3.0, 1.5, 0.5], size=e.shape) * rng.choice([-1.0, 1.0], size=e.shape)
    x[:, ::group] = big
    x[:, 1::group] = small
    bits = oracle_lib.f32_to_bf16(x)
    assert (oracle_lib.bf16_to_f32(bits) == x).all()  # every input is exactly a bf16 value
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(bits, group))
    for rows in (slice(0, 1000), slice(0, m)):  # one workgroup per row (<= 1024 rows), then registers per row
        q, s = rotate_quant(to_dev_bf16(bits[rows]), group)
        np.testing.assert_array_equal(s.cpu().numpy(), sx[rows])
        np.testing.assert_array_equal(q.cpu().numpy(), xq[rows])
    # the case mix holds: most rotated values were rounded, and a quarter of them sat exactly halfway
    xr = oracle_lib.bf16_to_f32(oracle_lib.rotate(bits, group)).astype(np.float64)
    exact = (x.astype(np.float64).reshape(m, k // group, group) @ oracle_lib.regular_hadamard(group)).reshape(m, k)
    nz = exact != 0
    assert (xr[nz] != exact[nz]).mean() > 0.5
    half_units = np.abs(exact[nz]) / np.exp2(np.floor(np.log2(np.abs(exact[nz]))) - 8)
    assert (half_units % 2 == 1).mean() > 0.2


@pytest.mark.parametrize("group", [4, 16, 64, 256])
def test_rotate_quant_many_rows_every_group(oracle_lib, group):
    """The register-resident layout for each butterfly depth (natural order up to G = 16, transposed for 64, 256)."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    inp = oracle_lib.make_inputs(1031, 3072, 8, group, outlier_frac=0.01, outlier_scale=20.0, seed=group)
    q, s = rotate_quant(to_dev_bf16(inp["x"]), group)
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(inp["x"], group))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)


def test_rotate_quant_zero_rows_wide_spans_and_strides(oracle_lib):
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    rng = np.random.default_rng(77)
    x = rng.standard_normal((24, 1024)) * np.exp2(rng.integers(-30, 4, size=(24, 1024)))
    x[3] = 0.0
    x[5, :] = 1e-30
    x[6, ::2] = 3e4
    bits = oracle_lib.f32_to_bf16(x.astype(np.float32))
    padded = np.zeros((24, 1024 + 64), dtype=np.uint16)
    padded[:, :1024] = bits
    xt = to_dev_bf16(padded)[:, :1024]  # row stride 1088 elements
    q, s = rotate_quant(xt, 256)
    sx, xq = oracle_lib.quantize(oracle_lib.rotate(bits, 256))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)
    assert s[3].item() == np.float32(np.float32(1e-12) / np.float32(127.0)) and not q[3].any()


# ------------------------------------------------------------------------------------------------ the whole layer


@pytest.mark.parametrize("name", [n for n in FIXTURES if n != "composition"] + ["composition"])
def test_layer_matches_reference_golden_bitwise(oracle_lib, name):
    f = load_fixture(name)
    layer = make_layer(f, f["K"], f["N"], f["G"])
    with torch.no_grad():
        y = layer(to_dev_bf16(f["x"]))
    assert y.dtype == torch.bfloat16 and y.shape == (f["M"], f["N"])
    np.testing.assert_array_equal(bits_of(y), f["y"])


def test_layer_accepts_leading_dims_and_casts_back(oracle_lib):
    inp = oracle_lib.make_inputs(35, 128, 96, 16, outlier_frac=0.0, seed=3, weight_dist="quantized")
    layer = make_layer(inp, 128, 96, 16)
    x = to_dev_bf16(inp["x"]).float().reshape(5, 7, 128)
    with torch.no_grad():
        y = layer(x)
    assert y.shape == (5, 7, 96) and y.dtype == torch.float32
    ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], 16)["y"]
    np.testing.assert_array_equal(bits_of(y.reshape(35, 96).to(torch.bfloat16)), ref)


def test_int8_linear_matches_dense():
    """tests/test_int8.py:51-63 on the device: relative-norm error < 0.02 against the dense fp32 linear."""
    from hyperflow_h3_flash_amd import Int8RotLinear
    from oracle import oracle

    torch.manual_seed(0)
    weight = torch.randn(96, 128) * 0.05
    x = torch.randn(5, 7, 128)
    layer = Int8RotLinear(128, 96, group=16)
    q, ws = oracle.quantize_weight(weight.double().numpy(), 16)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(q))
        layer.wscale.copy_(torch.from_numpy(ws))
    layer = layer.to(DEV)
    with torch.no_grad():
        y = layer(x.to(DEV)).cpu()
    reference = x @ weight.T
    assert y.shape == (5, 7, 96) and y.dtype == x.dtype
    error = (y.float() - reference).norm() / reference.norm()
    assert error < 0.02, error


def test_empty_and_single_row(oracle_lib):
    inp = oracle_lib.make_inputs(1, 256, 64, 256, seed=8)
    layer = make_layer(inp, 256, 64, 256)
    with torch.no_grad():
        y1 = layer(to_dev_bf16(inp["x"]))
        y0 = layer(torch.zeros(0, 256, dtype=torch.bfloat16, device=DEV))
    assert y0.shape == (0, 64)
    np.testing.assert_array_equal(bits_of(y1), oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"],
                                                                         256)["y"])


def test_odd_n_and_output_stride(oracle_lib):
    from hyperflow_h3_flash_amd import _native

    inp = oracle_lib.make_inputs(70, 512, 97, 64, seed=21)
    ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], 64)
    x = to_dev_bf16(inp["x"])
    w = torch.from_numpy(inp["qweight"]).to(DEV)
    ws = torch.from_numpy(inp["wscale"]).to(DEV)
    q = torch.empty(70, 512, dtype=torch.int8, device=DEV)
    s = torch.empty(70, dtype=torch.float32, device=DEV)
    y = torch.full((70, 101), -1, dtype=torch.int16, device=DEV)  # row stride 101, canary in the padding
    lib = _native.library()
    st = lib.hf_convrot_linear(x.data_ptr(), 512, w.data_ptr(), 512, ws.data_ptr(), None, 0, None, 0, 0, None, 64,
                               q.data_ptr(), s.data_ptr(), None, y.data_ptr(), 101, 70, 97, 512,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    yh = y.cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(yh[:, :97], ref["y"])
    assert (yh[:, 97:] == 0xFFFF).all()


# ------------------------------------------------------------------------------------- low-rank + bias extension


def test_lowrank_bias_extension_against_the_reference_composition(oracle_lib):
    f = load_fixture("composition")
    layer = make_layer(f, f["K"], f["N"], f["G"], rank=f["down"].shape[0], bias=True)
    with torch.no_grad():
        layer.down.weight.copy_(to_dev_bf16(f["down"]))
        layer.up.weight.copy_(to_dev_bf16(f["up"]))
        layer.bias.copy_(to_dev_bf16(f["bias"]))
        y = layer(to_dev_bf16(f["x"]))
    got = oracle_lib.bf16_to_f32(bits_of(y))
    # against the reference's bf16 composition (written by its modules), elementwise: every element within the
    # composition's rounding bound plus the device's fp32 summation slack, >= 99.5 % within one bf16 step, and
    # max |y - y_ref| / max |y_ref| <= 1e-2
    extra = device_lowrank_slack(f["x"], f["down"], f["u"], f["up"], f["y"], f["bias"])
    check_against_composition(bits_of(y), f["y"], f["lowrank"], f["bias"], f["y_composed"], extra=extra)
    # against the fused definition (fp32 sum, one rounding): within one bf16 ulp, elementwise
    out = oracle_lib.convrot_linear(f["x"], f["qweight"], f["wscale"], f["G"])
    u = oracle_lib.lowrank_down(f["x"], f["down"])
    fused = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(out["acc"], out["sx"], f["wscale"], u, f["up"],
                                                             f["bias"]))
    assert (np.abs(got - fused) <= np.abs(fused) * 2.0**-7 + 1e-6).all()


@pytest.mark.parametrize("rank", [8, 24, 32, 64, 136])
def test_lowrank_down_matches_oracle(oracle_lib, rank):
    from hyperflow_h3_flash_amd.int8 import lowrank_down

    inp = oracle_lib.make_inputs(100, 1024, 16, 256, rank=rank, seed=rank)
    u = lowrank_down(to_dev_bf16(inp["x"]), to_dev_bf16(inp["down"]))
    got = oracle_lib.bf16_to_f32(bits_of(u))
    ref = oracle_lib.bf16_to_f32(oracle_lib.lowrank_down(inp["x"], inp["down"]))
    # fp32 accumulation vs the oracle's exactly rounded sum
    assert within_fp32_sum_bound(got, ref, oracle_lib.bf16_to_f32(inp["x"]), oracle_lib.bf16_to_f32(inp["down"]))
    assert (got == ref).mean() > 0.99


@pytest.mark.parametrize("m,rank", [(32768, 64), (37710, 64), (45000, 32), (60001, 64), (70000, 136)])
def test_lowrank_down_many_rows_on_sampled_rows(oracle_lib, m, rank):
    """Row counts that take 4 to 8 waves per workgroup (one round of workgroups up to 256 x 256 rows, more rounds
    past it), a ragged last workgroup and a rank split over two launches; the oracle checks a seeded sample of rows
    and the last rows."""
    from hyperflow_h3_flash_amd.int8 import lowrank_down

    k = 1024
    gen = torch.Generator(device=DEV).manual_seed(m + rank)
    x = torch.randn(m, k, device=DEV, generator=gen).to(torch.bfloat16)
    down = (torch.randn(rank, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    u = lowrank_down(x, down)
    torch.cuda.synchronize()
    rows = np.concatenate([np.sort(np.random.default_rng(m).choice(m, size=24, replace=False)), np.arange(m - 8, m)])
    got = oracle_lib.bf16_to_f32(bits_of(u[rows]))
    ref = oracle_lib.bf16_to_f32(oracle_lib.lowrank_down(bits_of(x[rows]), bits_of(down)))
    assert within_fp32_sum_bound(got, ref, x[rows].float().cpu().numpy(), down.float().cpu().numpy())
    assert (got == ref).mean() > 0.99


# ------------------------------------------------------------------------------------------- benchmark-size shapes


@pytest.mark.parametrize("m,k,n", [(4096, 5120, 2048), (32768, 5120, 15360),
                                   # the model's own linears: q/k/v, out, the gated FFN's up and down, fused q/k/v
                                   (4099, 5376, 7168), (4099, 7168, 5376), (2053, 5376, 28672), (2053, 14336, 5376),
                                   (4099, 5376, 21504)])
def test_benchmark_shapes_on_sampled_rows(oracle_lib, m, k, n):
    """The full-size layer on the device; the oracle checks a seeded sample of rows (rows are independent), and
    size-independent properties are checked on every row. Also the model's own linear shapes (hidden 5376, attention
    7168, feed-forward 2 x 14336) with a ragged row count."""
    from hyperflow_h3_flash_amd import Int8RotLinear
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    g = 256
    gen = torch.Generator(device=DEV).manual_seed(m + n)
    x = torch.randn(m, k, device=DEV, generator=gen)
    cols = torch.randperm(k, device=DEV, generator=gen)[: max(1, k // 200)]
    x[:, cols] *= 30.0
    x = x.to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen)
    ws = torch.rand(n, device=DEV, generator=gen) * 9e-3 + 1e-3
    layer = Int8RotLinear(k, n, g).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(w)
        layer.wscale.copy_(ws)
        y = layer(x)
        q, s = rotate_quant(x, g)
    torch.cuda.synchronize()
    # every row: the absmax element quantizes to +-127 and no code leaves [-127, 127]
    assert int(q.abs().amax(dim=1).min()) == 127 and int(q.min()) >= -127
    rows = np.sort(np.random.default_rng(m).choice(m, size=12, replace=False))
    xb = bits_of(x[rows])
    ref = oracle_lib.convrot_linear(xb, w.cpu().numpy(), ws.cpu().numpy(), g)
    np.testing.assert_array_equal(s[rows].cpu().numpy(), ref["sx"])
    np.testing.assert_array_equal(q[rows].cpu().numpy(), ref["xq"])
    np.testing.assert_array_equal(bits_of(y[rows]), ref["y"])


def test_q_k_v_share_one_quantization(monkeypatch, oracle_lib):
    """tests/test_int8.py:149-173 on the device."""
    from hyperflow_h3_flash_amd import Int8RotLinear
    from hyperflow_h3_flash_amd.int8 import _kernels

    kernels = _kernels()
    calls = []
    rotate_quant = kernels.rotate_quant
    monkeypatch.setattr(kernels, "rotate_quant", lambda *a: calls.append(1) or rotate_quant(*a))
    layers = []
    for seed in range(3):
        inp = oracle_lib.make_inputs(1000, 1024, 512, 256, seed=seed, outlier_frac=0.01, outlier_scale=30.0,
                                     weight_dist="quantized")
        layers.append(make_layer(inp, 1024, 512, 256))
        if seed == 0:
            x = to_dev_bf16(inp["x"])
    to_q, to_k, to_v = layers
    to_q.keep_input = to_k.keep_input = True
    with torch.no_grad():
        shared = [to_q(x), to_k(x), to_v(x)]
        assert len(calls) == 1 and not Int8RotLinear._last_input
        to_q.keep_input = to_k.keep_input = False
        separate = [to_q(x), to_k(x), to_v(x)]
        assert len(calls) == 4
        for a, b in zip(shared, separate):
            assert torch.equal(a, b)
        to_q.keep_input = True
        to_q(x)
        x.mul_(2)
        to_k(x)
        to_q(x)
        to_k(x.clone())
    assert len(calls) == 8
    Int8RotLinear._last_input.clear()
