"""The feed-forward activations fused into the INT8 GEMM epilogue: tanh-GELU on the bf16 linear output, and the
gated feed-forward's SwiGLU (hidden * silu(gate) of the output's two halves, the output half as wide).

Bars: the fused output is the oracle's tanh-GELU (torch's formula in fp32, pinned against torch in test_oracle.py)
of the same layer's unfused output: within 1e-3 of the output's maximum everywhere, and bitwise on at least 99.9 %
of the elements whose input is >= -3. Below -3 the formula's `1 + tanh(u)` cancels (tanh is within 1e-4 of -1), so
the last fp32 bits of tanh, which differ between any two implementations (the device uses exp2 and a reciprocal,
torch its own tanh), decide the bf16 rounding of values below 1e-2 in magnitude. With the low-rank branch and a
bias: within 1e-2 (max |y - y_ref| / max |y_ref|) of the reference's module composition followed by the
activation. Every GEMM path is covered: few-row split K and the skinny kernel (through `int8_matmul`, which passes a
workspace), and the 256 x 256 tile kernel at the same shapes (through the C ABI with no workspace).

SwiGLU bars: the fused output is the oracle's SwiGLU (torch's composition, pinned bitwise in test_oracle.py) of the
same layer's unfused output: bitwise on at least 99.9 % of the elements and within 2^-6 of each element's value
everywhere (the device's SiLU uses exp2 and a reciprocal, so its fp32 value can differ from torch's in the last bits
and, rarely, round to the neighbouring bf16 value). Both half orders, every GEMM path, ranks 32, 64 (operands through
LDS) and 96 (from global memory).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

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


def act_linear(q, w, sx, ws, kw, activation, split):
    """The fused layer through `int8_matmul` (which hands the library a workspace, so few-row shapes take the split-K
    or skinny path) or, with `split=False`, through the C ABI with no workspace: the 256 x 256 tile kernel at any
    shape."""
    from hyperflow_h3_flash_amd import _native
    from hyperflow_h3_flash_amd.int8 import ACTIVATIONS, int8_matmul

    if split:
        return int8_matmul(q, w, sx, ws, activation=activation, **kw)
    lib = _native.library()
    m, k = q.shape
    n = w.shape[0]
    code = ACTIVATIONS[activation]
    y = torch.full((m, n // 2 if code >= 2 else n), -1, device=DEV, dtype=torch.int16).view(torch.bfloat16)
    u, up, bias = kw.get("u"), kw.get("up"), kw.get("bias")
    r = 0 if u is None else u.shape[1]

    def ptr(t):
        return None if t is None else ctypes.c_void_p(t.data_ptr())

    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    status = lib.hf_int8_linear_act_ws(ptr(q), k, ptr(w), k, ptr(sx), ptr(ws), ptr(u), r, ptr(up), r, r, ptr(bias),
                                       code, ptr(y), y.shape[1], m, n, k, None, 0, stream)
    assert status == 0
    return y


def check_gelu(got_bits, pre_bits, lib):
    """`got_bits` against the oracle's activation of the pre-activation bf16 values `pre_bits`."""
    ref_bits = lib.gelu_tanh(pre_bits)
    got, ref = lib.bf16_to_f32(got_bits), lib.bf16_to_f32(ref_bits)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    well_conditioned = lib.bf16_to_f32(pre_bits) >= -3.0
    exact = (got_bits == ref_bits)[well_conditioned].mean()
    assert rel <= 1e-3, (rel, exact)
    assert exact >= 0.999, (rel, exact)


# (M, K, N): 256 x 256 tiles with a ragged edge, few rows (split K), at most 64 rows (skinny kernel)
SHAPES = [(600, 1024, 700), (200, 2048, 512), (100, 1024, 300), (40, 1024, 300), (1, 512, 64)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("rank,bias", [(0, False), (64, True), (32, False)])
@pytest.mark.parametrize("split", [True, False])
def test_gelu_epilogue_is_gelu_of_the_linear_output(oracle_lib, m, k, n, rank, bias, split):
    from hyperflow_h3_flash_amd.int8 import int8_matmul, lowrank_down, rotate_quant

    inp = oracle_lib.make_inputs(m, k, n, 256, rank=rank, bias=bias, outlier_frac=0.01, outlier_scale=20.0,
                                 seed=m + k + n + rank)
    x = to_dev_bf16(inp["x"])
    w = torch.from_numpy(inp["qweight"]).to(DEV)
    ws = torch.from_numpy(inp["wscale"]).to(DEV)
    q, sx = rotate_quant(x, 256)
    kw = {}
    if rank:
        kw = dict(u=lowrank_down(x, to_dev_bf16(inp["down"])), up=to_dev_bf16(inp["up"]))
    if bias:
        kw["bias"] = to_dev_bf16(inp["bias"])
    plain = int8_matmul(q, w, sx, ws, **kw)
    fused = act_linear(q, w, sx, ws, kw, "gelu_tanh", split)
    torch.cuda.synchronize()
    check_gelu(bits_of(fused), bits_of(plain), oracle_lib)


def test_gelu_layer_against_the_reference_composition(oracle_lib):
    """Int8RotLinear(activation="gelu_tanh") with the low-rank branch and a bias against gelu(Int8RotLinear(x) +
    LowRankLinear(x) + bias), the reference modules composed in bf16."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    m, k, n, g, r = 300, 1024, 520, 256, 64
    inp = oracle_lib.make_inputs(m, k, n, g, rank=r, bias=True, outlier_frac=0.005, outlier_scale=30.0, seed=7)
    layer = Int8RotLinear(k, n, g, rank=r, bias=True, activation="gelu_tanh").to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        layer.down.weight.copy_(to_dev_bf16(inp["down"]))
        layer.up.weight.copy_(to_dev_bf16(inp["up"]))
        layer.bias.copy_(to_dev_bf16(inp["bias"]))
        y = layer(to_dev_bf16(inp["x"]))
    out = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    comp = oracle_lib.composition(out["y"], inp["x"], inp["down"], inp["up"], inp["bias"])
    ref = oracle_lib.bf16_to_f32(oracle_lib.gelu_tanh(comp))
    got = oracle_lib.bf16_to_f32(bits_of(y))
    tolerance = 1e-2  # max |y - y_ref| / max |y_ref| against the reference's bf16 composition + activation
    assert np.abs(got - ref).max() / np.abs(ref).max() <= tolerance


def test_gelu_layer_without_extension_is_gelu_of_the_reference_output(oracle_lib):
    """No low-rank branch, no bias: the activation of the reference's bitwise output."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    m, k, n, g = 257, 512, 300, 64
    inp = oracle_lib.make_inputs(m, k, n, g, seed=11)
    layer = Int8RotLinear(k, n, g, activation="gelu_tanh").to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        y = layer(to_dev_bf16(inp["x"]))
    check_gelu(bits_of(y), oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)["y"], oracle_lib)


def check_swiglu(got_bits, pre_bits, lib, gate_first=False):
    """`got_bits` [M, F] against the oracle's SwiGLU of the pre-activation bf16 values `pre_bits` [M, 2F]."""
    ref_bits = lib.swiglu(pre_bits, gate_first=gate_first)
    assert got_bits.shape == ref_bits.shape
    got, ref = lib.bf16_to_f32(got_bits), lib.bf16_to_f32(ref_bits)
    exact = (got_bits == ref_bits).mean()
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0**-6 + 1e-37).all(), np.abs(got - ref).max()
    assert exact >= 0.999, exact


# (M, K, N), N a multiple of 32: whole tiles, a ragged row and column edge, few rows (split K), the skinny kernel
GLU_SHAPES = [(600, 1024, 768), (300, 512, 544), (200, 2048, 512), (100, 1024, 320), (40, 1024, 320), (1, 512, 64)]


@pytest.mark.parametrize("m,k,n", GLU_SHAPES)
@pytest.mark.parametrize("rank,bias", [(0, False), (64, True), (32, False), (96, True)])
@pytest.mark.parametrize("gate_first", [False, True])
@pytest.mark.parametrize("split", [True, False])
def test_swiglu_epilogue_is_swiglu_of_the_linear_output(oracle_lib, m, k, n, rank, bias, gate_first, split):
    from hyperflow_h3_flash_amd.int8 import int8_matmul, lowrank_down, rotate_quant

    inp = oracle_lib.make_inputs(m, k, n, 256, rank=rank, bias=bias, outlier_frac=0.01, outlier_scale=20.0,
                                 seed=m + k + n + rank + gate_first)
    x = to_dev_bf16(inp["x"])
    w = torch.from_numpy(inp["qweight"]).to(DEV)
    ws = torch.from_numpy(inp["wscale"]).to(DEV)
    q, sx = rotate_quant(x, 256)
    kw = {}
    if rank:
        kw = dict(u=lowrank_down(x, to_dev_bf16(inp["down"])), up=to_dev_bf16(inp["up"]))
    if bias:
        kw["bias"] = to_dev_bf16(inp["bias"])
    plain = int8_matmul(q, w, sx, ws, **kw)
    fused = act_linear(q, w, sx, ws, kw, "swiglu_gate_first" if gate_first else "swiglu", split)
    torch.cuda.synchronize()
    assert fused.shape == (m, n // 2)
    check_swiglu(bits_of(fused), bits_of(plain), oracle_lib, gate_first)


def test_swiglu_layer_against_the_reference_composition(oracle_lib):
    """Int8RotLinear(activation="swiglu") with the low-rank branch and a bias against swiglu(Int8RotLinear(x) +
    LowRankLinear(x) + bias), the reference modules composed in bf16."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    m, k, n, g, r = 300, 1024, 576, 256, 64
    inp = oracle_lib.make_inputs(m, k, n, g, rank=r, bias=True, outlier_frac=0.005, outlier_scale=30.0, seed=17)
    layer = Int8RotLinear(k, n, g, rank=r, bias=True, activation="swiglu").to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        layer.down.weight.copy_(to_dev_bf16(inp["down"]))
        layer.up.weight.copy_(to_dev_bf16(inp["up"]))
        layer.bias.copy_(to_dev_bf16(inp["bias"]))
        y = layer(to_dev_bf16(inp["x"]).reshape(3, 100, k))
    assert y.shape == (3, 100, n // 2)
    out = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    comp = oracle_lib.composition(out["y"], inp["x"], inp["down"], inp["up"], inp["bias"])
    ref = oracle_lib.bf16_to_f32(oracle_lib.swiglu(comp))
    got = oracle_lib.bf16_to_f32(bits_of(y.reshape(m, n // 2)))
    # max |y - y_ref| / max |y_ref| against the reference's bf16 composition + activation: the output is the product
    # of two linear outputs, each within the linear's 1e-2 bar (the fused epilogue rounds once where the composition
    # rounds three times), so the product's bar is twice that.
    tolerance = 2e-2
    assert np.abs(got - ref).max() / np.abs(ref).max() <= tolerance
    # and each half of the unfused layer is within the linear's own bar of the composition
    layer.activation = None
    with torch.no_grad():
        plain = bits_of(layer(to_dev_bf16(inp["x"])))
    lin, lin_ref = oracle_lib.bf16_to_f32(plain), oracle_lib.bf16_to_f32(comp)
    assert np.abs(lin - lin_ref).max() / np.abs(lin_ref).max() <= 1e-2
    check_swiglu(bits_of(y.reshape(m, n // 2)), plain, oracle_lib)


def test_swiglu_layer_without_extension_is_swiglu_of_the_reference_output(oracle_lib):
    """No low-rank branch, no bias: SwiGLU of the reference's bitwise output."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    m, k, n, g = 257, 512, 320, 64
    inp = oracle_lib.make_inputs(m, k, n, g, seed=21)
    layer = Int8RotLinear(k, n, g, activation="swiglu").to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
        y = layer(to_dev_bf16(inp["x"]))
    check_swiglu(bits_of(y), oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)["y"], oracle_lib)


def test_swiglu_silu_on_every_bf16_gate_value(oracle_lib):
    """SiLU on every finite normal bf16 value, read straight off the fused output: the hidden half is exactly 1 (zero
    weight rows plus a bias of 1) and the gate half's bf16 values are built exactly from integer accumulators and
    power-of-two scales: value bits (m << 8) | j from row m and column j (acc = 128 + j % 128, sx[m] = +-2^(2 (m %
    128) - 134), wscale[j] = 2^(j // 128)); columns 256..511 repeat them scaled by 2^-64 and rows m % 128 < 4 are
    scaled by 2^64, so the smallest exponents come out in range. Bar: the fused output equals the oracle's SwiGLU of
    the unfused output bitwise, but for at most 8 values (the oracle's SiLU and torch's differ on at most 8 bf16
    values). Both the tile kernel (256 rows) and the skinny split-K path (64-row slices) are run."""
    from hyperflow_h3_flash_amd.int8 import int8_matmul

    m_rows, f, k = 256, 512, 32
    q = np.zeros((m_rows, k), np.int8)
    q[:, 0:3] = 1
    w = np.zeros((2 * f, k), np.int8)
    j = np.arange(f)
    w[f:, 0] = 64
    w[f:, 1] = 64
    w[f:, 2] = j % 128  # acc = 128 + j % 128
    m = np.arange(m_rows)
    e = 2 * (m % 128) - 134
    e = np.where(m % 128 < 4, e + 64, e)
    sx = np.where(m >= 128, -1.0, 1.0) * np.exp2(e.astype(np.float64))
    sw = np.ones(2 * f)
    sw[f:] = np.exp2((j % 256 // 128) - np.where(j >= 256, 64, 0))
    bias = np.zeros(2 * f, np.float32)
    bias[:f] = 1.0
    dq, dw = torch.from_numpy(q).to(DEV), torch.from_numpy(w).to(DEV)
    dsx = torch.from_numpy(sx.astype(np.float32)).to(DEV)
    dsw = torch.from_numpy(sw.astype(np.float32)).to(DEV)
    db = to_dev_bf16(oracle_lib.f32_to_bf16(bias))
    plain = bits_of(int8_matmul(dq, dw, dsx, dsw, bias=db))
    fused_tiles = bits_of(act_linear(dq, dw, dsx, dsw, {"bias": db}, "swiglu", split=False))
    fused_rows = np.concatenate([bits_of(int8_matmul(dq[i:i + 64], dw, dsx[i:i + 64], dsw, bias=db,
                                                     activation="swiglu")) for i in range(0, m_rows, 64)])
    gate = plain[:, f:]
    normal = np.arange(65536, dtype=np.uint16)
    normal = normal[((normal >> 7) & 0xFF != 0) & ((normal >> 7) & 0xFF != 0xFF)]
    assert np.isin(normal, gate).all(), "the gate half misses some bf16 values"
    assert (plain[:, :f] == 0x3F80).all()  # hidden half exactly 1.0
    ref = oracle_lib.swiglu(plain)
    finite = np.isfinite(oracle_lib.bf16_to_f32(gate))
    for fused in (fused_tiles, fused_rows):
        assert ((fused != ref) & finite).sum() <= 8
