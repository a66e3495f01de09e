"""The reference's GPU-kernel arithmetic for the rotation + quantization (int8.py:194-262: the rotated value in fp32,
a reciprocal multiply), selected with `set_arithmetic_options(rotate_quant="f32_recip")` or the C ABI's
`hf_rotate_quant_ex(..., HF_ROTATE_F32_RECIP, ...)`.

Bar: bitwise equal codes and scales to the oracle's restatement (`rotate_f32` + `quantize_recip`, pinned by exact
arithmetic in test_oracle.py), and the layer's output bitwise the oracle's epilogue of those codes. Parity against the
reference's Triton kernels themselves is not checked here: they need CUDA.
"""

from __future__ import annotations

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


# Rows of up to 20 tiles of 1024 are held in registers (1 to 4 waves per row, ragged last waves); wider rows take the
# two-pass kernel. Group 1024 adds a radix-4 stage after a second transpose.
_F32_CASES = [(g, m, k) for g in (4, 16, 64, 256, 1024)
              for m, k in ((1, 256), (7, 1280), (65, 2304), (130, 5120), (1029, 5376), (33, 14336), (9, 20480),
                           (3, 21504), (2, 98304))
              if k % g == 0]


@pytest.mark.parametrize("group,m,k", _F32_CASES)
def test_f32_recip_matches_the_oracle(oracle_lib, group, m, k):
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    print(f"f32_recip rotation M={m} K={k} G={group}", flush=True)
    inp = oracle_lib.make_inputs(m, k, 8, group, outlier_frac=0.01, outlier_scale=30.0, seed=m + k + group)
    q, s = rotate_quant(to_dev_bf16(inp["x"]), group, arithmetic="f32_recip")
    sx, xq = oracle_lib.quantize_recip(oracle_lib.rotate_f32(inp["x"], group))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)


def test_f32_recip_zero_rows_wide_spans_and_strides(oracle_lib):
    """Zero rows, values spanning many binades (the exact-sum claim), and a row stride wider than K."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    rng = np.random.default_rng(5)
    m, k, g = 40, 1024, 256
    x = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-20, 12, size=(m, k)))).astype(np.float32)
    x[3] = 0.0
    x[7, ::5] = 0.0
    bits = oracle_lib.f32_to_bf16(x)
    wide = np.zeros((m, k + 64), dtype=np.uint16)
    wide[:, :k] = bits
    xd = to_dev_bf16(wide)[:, :k]
    q, s = rotate_quant(xd, g, arithmetic="f32_recip")
    sx, xq = oracle_lib.quantize_recip(oracle_lib.rotate_f32(bits, g))
    np.testing.assert_array_equal(s.cpu().numpy(), sx)
    np.testing.assert_array_equal(q.cpu().numpy(), xq)
    assert not q[3].any()


def test_layer_under_f32_recip_is_the_oracle_epilogue_of_its_codes(oracle_lib):
    """The module with the option set: codes, scales and the bitwise output follow the GPU-kernel arithmetic; the
    default (torch path) comes back when the option is reset."""
    from hyperflow_h3_flash_amd import Int8RotLinear, set_arithmetic_options

    m, k, n, g = 300, 2048, 520, 256
    inp = oracle_lib.make_inputs(m, k, n, g, outlier_frac=0.005, outlier_scale=30.0, seed=9)
    layer = Int8RotLinear(k, n, g).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.from_numpy(inp["qweight"]))
        layer.wscale.copy_(torch.from_numpy(inp["wscale"]))
    x = to_dev_bf16(inp["x"])
    try:
        set_arithmetic_options(rotate_quant="f32_recip")
        with torch.no_grad():
            y = layer(x)
    finally:
        set_arithmetic_options(rotate_quant="bf16_div")
    sx, xq = oracle_lib.quantize_recip(oracle_lib.rotate_f32(inp["x"], g))
    want = oracle_lib.epilogue(oracle_lib.int8_gemm(xq, inp["qweight"]), sx, inp["wscale"])
    np.testing.assert_array_equal(bits_of(y), want)
    with torch.no_grad():
        y_torch_path = layer(x)
    np.testing.assert_array_equal(bits_of(y_torch_path),
                                  oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)["y"])


def test_f32_recip_at_the_benchmark_size_on_sampled_rows(oracle_lib):
    """M=32768, K=5120 on the device; the oracle checks a seeded sample of rows, and every row reaches +-127."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    m, k, g = 32768, 5120, 256
    gen = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn(m, k, device=DEV, generator=gen)
    x[:, torch.randperm(k, device=DEV, generator=gen)[: k // 200]] *= 30.0
    x = x.to(torch.bfloat16)
    q, s = rotate_quant(x, g, arithmetic="f32_recip")
    torch.cuda.synchronize()
    assert int(q.abs().amax(dim=1).min()) == 127 and int(q.min()) >= -127
    rows = np.sort(np.random.default_rng(1).choice(m, size=16, replace=False))
    sx, xq = oracle_lib.quantize_recip(oracle_lib.rotate_f32(bits_of(x[rows]), g))
    np.testing.assert_array_equal(s[rows].cpu().numpy(), sx)
    np.testing.assert_array_equal(q[rows].cpu().numpy(), xq)
